"""The rest of the Depthformer boundary through the C ABI:

  * depth_forward_full (model.cpp:243-268): the depth stack over k positions in
    one pass against the oracle's full pass (causal and not, default and
    explicit bias, k < rvq_depth), and against the device's own step chain;
  * precompute_{temporal,depth}_biases (model.cpp:302-320) equal to the
    oracle's bias rows, bit for bit in the model dtype;
  * temporal_step / depth_step with an explicit position_bias: the precomputed
    bias reproduces the implicit call bit for bit, and a random bias matches
    the oracle's step with the same bias (persistent and multi-kernel paths);
  * the cache reset (empty_{temporal,depth}_cache, model.cpp:275-300).
Tolerances: fp32 <= 1e-4, bf16 <= 2e-2, fp16 <= 5e-3 norm-wise relative error.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = {"fp32": 1e-4, "bf16": 2e-2, "fp16": 5e-3}


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.fixture(scope="module")
def tiny(gpu_available):
    import mrt_df
    import synth_bundle
    from oracle import depthformer_oracle as O
    cfg = mrt_df.Config.tiny()
    w = synth_bundle.make_weights(cfg, seed=21, norm_jitter=0.1)
    return dict(mrt_df=mrt_df, O=O, cfg=cfg, w=w, ocfg=O.DepthformerConfig(**dataclasses.asdict(cfg)))


def _dev(torch, a, dt):
    return torch.tensor(np.asarray(a, dtype=np.float32), device="cuda").to(dt)


@pytest.mark.parametrize("dtype", ["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("k,causal", [(16, True), (5, True), (16, False)])
def test_depth_forward_full_matches_oracle(tiny, dtype, k, causal):
    import torch
    mrt_df, O = tiny["mrt_df"], tiny["O"]
    m = mrt_df.Depthformer(tiny["w"], tiny["cfg"], dtype=dtype)
    st = m.new_state(max_frames=2)
    om = O.OracleDepthformer(tiny["w"], tiny["ocfg"], mode=dtype)
    rng = np.random.default_rng(k + 100 * causal)
    embs = om.P.r(rng.standard_normal((2, k, tiny["cfg"].d_model)).astype(np.float32))
    got = st.depth_forward_full(_dev(torch, embs, m.torch_dtype), causal=causal).cpu().numpy()
    exp = om.depth_forward_full(embs, causal=causal)
    errs = [rel(got[b, i], exp[b, i]) for b in range(2) for i in range(k)]
    assert max(errs) <= TOL[dtype], max(errs)
    # an explicit (H, k, k) bias: the default block reproduces the implicit call
    # bit for bit; a random one matches the oracle given the same bias
    blk = om.depth_bias(0, key_length=k, query_length=k)[0]
    again = st.depth_forward_full(_dev(torch, embs, m.torch_dtype), _dev(torch, blk, m.torch_dtype),
                                  causal=causal).cpu().numpy()
    np.testing.assert_array_equal(again, got)
    rb = om.P.r(rng.standard_normal(blk.shape).astype(np.float32))
    got_r = st.depth_forward_full(_dev(torch, embs, m.torch_dtype), _dev(torch, rb, m.torch_dtype),
                                  causal=causal).cpu().numpy()
    exp_r = om.depth_forward_full(embs, causal=causal, position_bias=rb[None])
    assert rel(got_r, exp_r) <= TOL[dtype]
    assert rel(got_r, got) > 10 * TOL[dtype]  # the bias was used
    st.close()
    m.close()


@pytest.mark.parametrize("dtype", ["fp32", "bf16", "fp16"])
def test_depth_forward_full_equals_step_chain_at_benchmark_dims(gpu_available, dtype):
    """model.h:27-31: the full causal pass is the parity target of the step
    chain.  Benchmark dims: the pass's logits at position i against the
    persistent depth_step chain fed the same embeddings, and against the oracle."""
    import torch
    import mrt_df
    import synth_bundle
    from oracle import depthformer_oracle as O
    cfg = mrt_df.Config.bench()
    w = synth_bundle.make_weights(cfg, seed=1234, threads=16)
    m = mrt_df.Depthformer(w, cfg, dtype=dtype)
    st = m.new_state(max_frames=1)
    om = O.OracleDepthformer(w, O.DepthformerConfig(**dataclasses.asdict(cfg)), mode=dtype)
    rng = np.random.default_rng(7)
    embs = om.P.r(rng.standard_normal((2, 16, cfg.d_model)).astype(np.float32))
    e = _dev(torch, embs, m.torch_dtype)
    full = st.depth_forward_full(e).cpu().numpy()
    steps = np.stack([st.depth_step(e[:, i].contiguous(), i).cpu().numpy() for i in range(16)], axis=1)
    exp = om.depth_forward_full(embs)
    for i in range(16):
        assert rel(full[:, i], exp[:, i]) <= TOL[dtype], i
        assert rel(full[:, i], steps[:, i]) <= TOL[dtype], i
    st.close()
    m.close()


@pytest.mark.parametrize("dtype", ["fp32", "bf16", "fp16"])
def test_precomputed_biases_equal_oracle(tiny, dtype):
    mrt_df, O = tiny["mrt_df"], tiny["O"]
    m = mrt_df.Depthformer(tiny["w"], tiny["cfg"], dtype=dtype)
    om = O.OracleDepthformer(tiny["w"], tiny["ocfg"], mode=dtype)
    for kind, n, ref in (("temporal", 50, om.temporal_bias), ("depth", 16, om.depth_bias)):
        got = m.precompute_biases(kind, n)
        for f in range(n):
            np.testing.assert_array_equal(got[f].float().cpu().numpy(), ref(f)[0, :, 0, :], err_msg=f"{kind} {f}")
    m.close()


@pytest.mark.parametrize("dtype", ["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("path", ["persistent", "layers"])
def test_steps_with_explicit_bias(tiny, monkeypatch, dtype, path):
    import torch
    mrt_df, O = tiny["mrt_df"], tiny["O"]
    if path == "layers":
        monkeypatch.setenv("MRT_DECODE_PATH", "layers")  # read when the state is created
    cfg = tiny["cfg"]
    m = mrt_df.Depthformer(tiny["w"], cfg, dtype=dtype)
    om = O.OracleDepthformer(tiny["w"], tiny["ocfg"], mode=dtype)
    rng = np.random.default_rng(3)
    S = cfg.max_encoder_length
    tok = rng.integers(2, cfg.vocab_size, size=(2, S)).astype(np.int32)
    tb, db = m.precompute_biases("temporal", 4), m.precompute_biases("depth", 4)
    a, b = m.new_state(max_frames=4), m.new_state(max_frames=4)
    a.encode(tok)
    b.encode(tok)
    enc = om.encode(tok)
    # state b's depth K/V past layer 0 depend on its biases: one oracle cache per state
    tcache, dca, dcb = om.empty_temporal_cache(), om.empty_depth_cache(), om.empty_depth_cache()
    H = cfg.num_heads
    for f in range(4):
        x = om.P.r(rng.standard_normal((2, cfg.d_model)).astype(np.float32))
        xd = _dev(torch, x, m.torch_dtype)
        ya = a.temporal_step(xd, f).float().cpu().numpy()
        yb = b.temporal_step(xd, f, position_bias=tb[f]).float().cpu().numpy()
        np.testing.assert_array_equal(ya, yb)
        # depth: a random bias on state b, the oracle with the same bias
        rb = om.P.r(rng.standard_normal((H, f + 1)).astype(np.float32))
        la = a.depth_step(xd, f).cpu().numpy()
        lb = b.depth_step(xd, f, position_bias=_dev(torch, rb, m.torch_dtype)).cpu().numpy()
        ea = om.depth_step(x[:, None], dca, f)
        eb = om.depth_step(x[:, None], dcb, f, position_bias=rb[None, :, None, :])
        assert rel(la, ea) <= TOL[dtype], f
        assert rel(lb, eb) <= TOL[dtype], f
        if f > 0:  # one key: softmax ignores the bias
            assert rel(lb, la) > TOL[dtype]  # the bias was used
        ot = om.temporal_step(x[:, None], enc, tcache, f)
        assert rel(ya, ot[:, 0]) <= TOL[dtype]
    a.close()
    b.close()
    m.close()


def test_reset_cache(tiny):
    import torch
    mrt_df = tiny["mrt_df"]
    cfg = tiny["cfg"]
    m = mrt_df.Depthformer(tiny["w"], cfg, dtype="fp32")
    st = m.new_state(max_frames=4)
    x = torch.zeros((2, cfg.d_model), dtype=torch.float32, device="cuda")
    for i in range(3):
        st.depth_step(x, i)
    st.reset_cache("depth")
    with pytest.raises(mrt_df.MrtError, match="cache holds 0 entries"):
        st.depth_step(x, 3)
    st.depth_step(x, 0)
    st.encode(np.full((2, cfg.max_encoder_length), 5, dtype=np.int32))
    st.temporal_step(x, 0)
    st.temporal_step(x, 1)
    st.reset_cache("temporal")
    with pytest.raises(mrt_df.MrtError, match="cache holds 0 entries"):
        st.temporal_step(x, 2)
    st.temporal_step(x, 0)
    with pytest.raises(KeyError):
        st.reset_cache("cross")
    st.close()
    m.close()
