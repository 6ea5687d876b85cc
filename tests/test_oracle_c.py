"""The C/OpenMP restatement (oracle/df_cpu.c) against the numpy oracle at the
tiny dims.  fp32: two independent restatements of model.cpp:226-659 and
decode.cpp:239-573 written separately must agree to float32 rounding -- the
decode steps with their caches at 1 thread and at several, the encoder, the
cross K/V projection and the whole teacher-forced and free-running loop
(slices, temporal outputs, frame means, draws).  bf16: the C restatement is
another bf16 evaluation rounding at the same op boundaries; it stays closer to
the numpy bf16 oracle than either is to fp32, its single-GEMM outputs (the
cross K/V) are bit-identical to numpy's nearly everywhere, and the frame means
(sums of the same bf16 rows) are bit-exact."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import depthformer_oracle as O
from oracle import df_cpu

import synth_bundle
from draw_check import assert_draws


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.fixture(scope="module")
def env():
    df_cpu.build()
    cfg = O.DepthformerConfig.tiny()
    w = synth_bundle.make_weights(cfg, seed=9, norm_jitter=0.2)
    return cfg, w


@pytest.mark.parametrize("threads", [1, 4])
def test_c_steps_equal_numpy_oracle(env, threads):
    cfg, w = env
    df_cpu.CpuDepthformer.set_threads(threads)
    om = O.OracleDepthformer(w, cfg, mode="fp32")
    cm = df_cpu.CpuDepthformer(w, cfg, max_frames=6)
    rng = np.random.default_rng(threads)
    enc_tokens = rng.integers(0, cfg.vocab_size, (2, cfg.max_encoder_length))
    enc = om.encode(enc_tokens)
    cm.set_cross(om.precompute_cross_kv(enc))
    tcache = om.empty_temporal_cache()
    for f in range(6):
        x = rng.standard_normal((2, 1, cfg.d_model)).astype(np.float32)
        exp = om.temporal_step(x, enc, tcache, f)
        got = cm.temporal_step(x, f)
        assert rel(got, exp[:, 0]) <= 1e-5, f
        dcache = om.empty_depth_cache()
        for l in range(cfg.rvq_depth):
            y = rng.standard_normal((2, 1, cfg.d_model)).astype(np.float32)
            full = om.depth_step(y, dcache, l)
            if l % 2:
                got = cm.depth_step(y, l)
                assert rel(got, full) <= 1e-5, (f, l)
            else:
                got = cm.depth_step(y, l, level=l, codebook=8, codec_offset=2)
                assert rel(got, full[:, 2 + 8 * l: 2 + 8 * (l + 1)]) <= 1e-5, (f, l)
        for i in range(cfg.num_depth_layers):
            assert rel(cm.dk[i], dcache[i]["k"]) <= 1e-5
            assert rel(cm.dv[i], dcache[i]["v"]) <= 1e-5
    for i in range(cfg.num_temporal_layers):
        assert rel(cm.tk[i], tcache[i]["k"]) <= 1e-5
        assert rel(cm.tv[i], tcache[i]["v"]) <= 1e-5


@pytest.fixture(scope="module")
def chunk(env):
    cfg, w = env
    df_cpu.CpuDepthformer.set_threads(4)
    rng = np.random.default_rng(77)
    tok = rng.integers(0, cfg.vocab_size, (2, cfg.max_encoder_length))
    F = 6
    teacher = (2 + 8 * np.arange(16)[None, :] + rng.integers(0, 8, (F, 16))).astype(np.int32)
    opts = O.GenerateOptions(num_frames=F, rvq_depth=16, temperature=1.1, top_k=4, guidance_weight=5.0, seed=3,
                             codebook_size=8, codec_offset=2)
    res = {}
    for mode in ("fp32", "bf16"):
        om = O.OracleDepthformer(w, cfg, mode=mode)
        cm = df_cpu.CpuDepthformer(w, cfg, max_frames=F, mode=mode)
        enc_n, enc_c = om.encode(tok), cm.encode(tok)
        cm.set_cross_from_encoder(enc_n)
        cross_n = om.precompute_cross_kv(enc_n)
        rn, rc = {}, {}
        O.generate_tokens(om, tok, opts, teacher=teacher, record=rn, enc_out=enc_n)
        tc = cm.generate(opts, teacher=teacher, record=rc)
        res[mode] = dict(enc=(enc_c, enc_n), cross=((cm.ck, cm.cv), cross_n), rn=rn, rc=rc, tc=tc, cm=cm)
    return cfg, w, tok, teacher, opts, res


def test_c_encoder_and_cross_kv_equal_numpy_fp32(chunk):
    *_, res = chunk
    r = res["fp32"]
    assert rel(*r["enc"]) <= 1e-5
    (ck, cv), cross_n = r["cross"]
    for i, (k, v) in enumerate(cross_n):
        assert rel(ck[i], k) <= 1e-5 and rel(cv[i], v) <= 1e-5, i


def test_c_generate_teacher_forced_equals_numpy_fp32(chunk):
    cfg, w, tok, teacher, opts, res = chunk
    r = res["fp32"]
    rn, rc = r["rn"], r["rc"]
    np.testing.assert_array_equal(r["tc"], teacher)
    assert rel(rc["slices"], rn["slices"]) <= 1e-5
    assert rel(rc["temporal_out"], rn["temporal_out"]) <= 1e-5
    np.testing.assert_array_equal(rc["frame_mean"], rn["frame_mean"])
    # every C draw is the numpy sampler's draw on the C's own logits (or an ulp tie)
    guided = np.array([[O.cfg_combine(rc["slices"][f, l], 5.0) for l in range(16)] for f in range(opts.num_frames)])
    assert_draws(O, rc["drawn"], guided, temperature=1.1, top_k=4, seed=3, offset=2, codebook=8, max_ties=2)
    for i in range(cfg.num_temporal_layers):  # temporal caches after the chunk: (2, H, frames, 64)
        assert rel(r["cm"].tk[i][:, :, :opts.num_frames], rn["temporal_cache"][i]["k"]) <= 1e-5
        assert rel(r["cm"].tv[i][:, :, :opts.num_frames], rn["temporal_cache"][i]["v"]) <= 1e-5


def test_c_generate_free_running_equals_numpy_fp32(env):
    cfg, w = env
    rng = np.random.default_rng(78)
    tok = rng.integers(0, cfg.vocab_size, (2, cfg.max_encoder_length))
    opts = O.GenerateOptions(num_frames=4, rvq_depth=16, temperature=1.1, top_k=4, guidance_weight=5.0, seed=9,
                             codebook_size=8, codec_offset=2)
    om = O.OracleDepthformer(w, cfg, mode="fp32")
    cm = df_cpu.CpuDepthformer(w, cfg, max_frames=4)
    enc = om.encode(tok)
    cm.set_cross_from_encoder(enc)
    rc = {}
    tc = cm.generate(opts, record=rc)
    np.testing.assert_array_equal(tc, rc["drawn"])
    # the numpy loop fed the C's tokens reproduces the C's logits, and each
    # C token is the numpy sampler's draw from them
    rn = {}
    O.generate_tokens(om, tok, opts, teacher=tc, record=rn, enc_out=enc)
    assert rel(rc["slices"], rn["slices"]) <= 1e-5
    guided = np.array([[O.cfg_combine(rn["slices"][f, l], 5.0) for l in range(16)] for f in range(4)])
    assert_draws(O, tc, guided, temperature=1.1, top_k=4, seed=9, offset=2, codebook=8, max_ties=2)


def test_c_bf16_is_a_bf16_evaluation_of_the_same_ops(chunk):
    *_, res = chunk
    r16, r32 = res["bf16"], res["fp32"]
    rn16, rc16, rn32 = r16["rn"], r16["rc"], r32["rn"]
    # rounding noise of the C bf16 run against numpy bf16 is below bf16 vs fp32
    gap = rel(rn16["slices"], rn32["slices"])
    assert rel(rc16["slices"], rn16["slices"]) <= 0.75 * gap, (rel(rc16["slices"], rn16["slices"]), gap)
    assert rel(rc16["slices"], rn32["slices"]) <= 1.5 * gap
    # one GEMM + rounding (the cross K/V): bit-identical nearly everywhere
    (ck, cv), cross_n = r16["cross"]
    same = np.mean([np.mean(ck[i] == k) for i, (k, _) in enumerate(cross_n)])
    assert same >= 0.99, same
    np.testing.assert_array_equal(rc16["frame_mean"], rn16["frame_mean"])
    assert rel(*r16["enc"]) <= 1e-2
