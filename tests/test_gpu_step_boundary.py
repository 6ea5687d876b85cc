"""The step-level boundary around temporal_step / depth_step, through the C ABI:

  * token_embedding()(ids) (model.h:127; the decode loop's feedback embedding,
    decode.cpp:366-368, 476-477): rows bit-equal to the oracle's embedding
    gather in the model dtype; an id outside the vocabulary is rejected;
  * position_embedding(seq_len) (model.cpp:215-224): the fp32 sinusoid rows
    within one ulp of sin / cos of the float32 angle evaluated in float64 (the
    closed form), and close to the oracle's table; seq_len past max_encoder_length
    fails as the reference's std::out_of_range does;
  * compile_for_inference (model.cpp:697-...): a compiled state and stream
    decode the same tokens as uncompiled ones, and leave caches and chunk
    index as they were;
  * the MRT_PROFILE_DECODE split (decode.cpp:529-565): with profiling on, the
    temporal, depth and draw times of the frame kernel are positive and add up
    to the decode section's event time within the launch gaps.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny(gpu_available):
    import mrt_df
    import synth_bundle
    from oracle import depthformer_oracle as O
    cfg = mrt_df.Config.tiny()
    w = synth_bundle.make_weights(cfg, seed=31, norm_jitter=0.1)
    return dict(mrt_df=mrt_df, O=O, cfg=cfg, w=w, ocfg=O.DepthformerConfig(**dataclasses.asdict(cfg)))


@pytest.mark.parametrize("dtype", ["fp32", "bf16", "fp16"])
def test_token_embedding_rows_equal_the_oracle_gather(tiny, dtype):
    mrt_df, O = tiny["mrt_df"], tiny["O"]
    m = mrt_df.Depthformer(tiny["w"], tiny["cfg"], dtype=dtype)
    om = O.OracleDepthformer(tiny["w"], tiny["ocfg"], mode=dtype)
    rng = np.random.default_rng(5)
    V = tiny["cfg"].vocab_size
    for n in (1, 2, 37, 5000):  # 5000 > the library's 4096-id staging chunk
        ids = rng.integers(0, V, n).astype(np.int32)
        ids[0] = V - 1
        got = m.token_embedding(ids).float().cpu().numpy()
        np.testing.assert_array_equal(got, om.P.r(om.embed(ids)))
    with pytest.raises(mrt_df.MrtError, match="token id out of range"):
        m.token_embedding(np.array([0, V], dtype=np.int32))
    with pytest.raises(mrt_df.MrtError, match="token id out of range"):
        m.token_embedding(np.array([-1], dtype=np.int32))
    m.close()


def test_position_embedding_is_the_fp32_sinusoid(tiny):
    mrt_df, O = tiny["mrt_df"], tiny["O"]
    cfg = tiny["cfg"]
    m = mrt_df.Depthformer(tiny["w"], cfg, dtype="bf16")
    S, D = cfg.max_encoder_length, cfg.d_model
    got = m.position_embedding(S).cpu().numpy()
    assert got.shape == (S, D) and got.dtype == np.float32
    half = D // 2
    f32 = np.float32
    # the float32 angles of model.cpp:62-74, evaluated in float64
    scale = f32(-np.log(f32(10000.0))) / f32(half - 1)
    div = np.array([f32(np.exp(np.float64(f32(i) * scale))) for i in range(half)], dtype=np.float32)
    ang = (np.arange(S, dtype=np.float32)[:, None] * div[None, :]).astype(np.float32).astype(np.float64)
    exact = np.concatenate([np.sin(ang), np.cos(ang)], axis=1)
    ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    assert (np.abs(got - exact) <= ulp).all()
    # the oracle's table takes div_term from numpy's float32 exp, which may be
    # an ulp (<= 2^-24 for div_term <= 1) away from the C library's expf: the
    # angle pos * div_term then moves by up to pos * 2^-23, and sin / cos with it
    table = O.sinusoidal_position_embedding(S, D)
    np.testing.assert_allclose(got, table, rtol=0, atol=(S - 1) * 2.0 ** -23 + 2.0 ** -22)
    np.testing.assert_array_equal(m.position_embedding(7).cpu().numpy(), got[:7])
    with pytest.raises(mrt_df.MrtError, match="seq_len exceeds max_encoder_length"):
        m.position_embedding(S + 1)
    m.close()


def _opts(mrt_df, F, seed, use_graph=True):
    return mrt_df.GenOptions(num_frames=F, rvq_depth=16, temperature=1.1, top_k=4, guidance_weight=5.0, seed=seed,
                             codebook_size=8, codec_offset=2, use_graph=use_graph)


def test_compiled_state_decodes_like_an_uncompiled_one(tiny):
    mrt_df = tiny["mrt_df"]
    cfg = tiny["cfg"]
    m = mrt_df.Depthformer(tiny["w"], cfg, dtype="bf16")
    rng = np.random.default_rng(3)
    tok = rng.integers(2, 130, size=(2, cfg.max_encoder_length)).astype(np.int32)
    F = 4
    ref = m.new_state(max_frames=F)
    exp = [ref.generate_tokens(tok if i == 0 else None, _opts(mrt_df, F, 11 + i)) for i in range(2)]
    ref.close()
    st = m.new_state(max_frames=F)
    st.compile_for_inference(_opts(mrt_df, F, 99))  # before any encode: an encoding of PAD ids, dropped
    with pytest.raises(mrt_df.MrtError, match="no encoder output"):
        st.generate_tokens(None, _opts(mrt_df, F, 11))
    got = [st.generate_tokens(tok if i == 0 else None, _opts(mrt_df, F, 11 + i)) for i in range(2)]
    for a, b in zip(got, exp):
        np.testing.assert_array_equal(a, b)
    # compiled after an encode: the encoder output and the next decode are unchanged
    st.compile_for_inference(_opts(mrt_df, F, 5))
    np.testing.assert_array_equal(st.generate_tokens(None, _opts(mrt_df, F, 12)), exp[1])
    st.close()
    m.close()


def test_compiled_stream_generates_like_an_uncompiled_one(tiny):
    mrt_df = tiny["mrt_df"]
    import system
    cfg = tiny["cfg"]
    m = mrt_df.Depthformer(tiny["w"], cfg, dtype="bf16")
    scfg = mrt_df.StreamConfig(chunk_frames=4, context_frames=10, codebook_size=8, encoder_codec_rvq_depth=4,
                               encoder_style_rvq_depth=6, decoder_codec_rvq_depth=16, mask_token=1, codec_offset=2)
    rng = np.random.default_rng(8)
    ctx = rng.integers(0, 8, (10, 16)).astype(np.int32)
    style = (2 + 16 * 8 + 8 * np.arange(6) + rng.integers(0, 8, 6)).astype(np.int32)
    assert style.max() < cfg.vocab_size
    outs = []
    for compiled in (False, True):
        s = mrt_df.Stream(m, scfg)
        s.set_context(ctx, 0)
        opts = mrt_df.ChunkOptions(temperature=1.1, top_k=4, guidance_weight=5.0, seed=21, pipeline_encoder=True,
                                   use_graph=True)
        if compiled:
            s.compile_for_inference(opts)
            got_ctx, idx = s.get_context()
            np.testing.assert_array_equal(got_ctx, ctx)
            assert idx == 0
        chunks = []
        for i in range(3):
            opts.seed = 21 + i
            chunks.append(s.generate_chunk(style, opts))
        outs.append(chunks)
        s.close()
    for (a_llm, a_rvq), (b_llm, b_rvq) in zip(*outs):
        np.testing.assert_array_equal(a_llm, b_llm)
        np.testing.assert_array_equal(a_rvq, b_rvq)
    assert system is not None
    m.close()


def test_decode_profile_splits_the_frame_kernel(tiny):
    mrt_df = tiny["mrt_df"]
    cfg = tiny["cfg"]
    m = mrt_df.Depthformer(tiny["w"], cfg, dtype="bf16")
    rng = np.random.default_rng(4)
    tok = rng.integers(2, 130, size=(2, cfg.max_encoder_length)).astype(np.int32)
    F = 8
    st = m.new_state(max_frames=F)
    plain = st.generate_tokens(tok, _opts(mrt_df, F, 7))
    p = st.decode_profile()
    assert p["temporal_ms"] == -1 and p["depth_ms"] == -1 and p["sample_ms"] == -1 and p["frames"] == 0
    assert p["total_ms"] > 0 and p["encoder_ms"] > 0 and p["bias_ms"] == 0
    st.set_profile(True)
    for use_graph in (False, True):
        got = st.generate_tokens(tok, _opts(mrt_df, F, 7, use_graph))
        np.testing.assert_array_equal(got, plain)  # the stamps change nothing
        p = st.decode_profile()
        assert p["frames"] == F
        assert p["temporal_ms"] > 0 and p["depth_ms"] > 0 and p["sample_ms"] > 0, p
        parts = p["temporal_ms"] + p["depth_ms"] + p["sample_ms"]
        # the stamps cover each frame launch from workgroup 0's start to its end;
        # the events add the noise table and the gaps between launches
        assert 0.5 * p["total_ms"] <= parts <= p["total_ms"], p
    st.close()
    m.close()
