"""Device-resident stream (the token half of System::generate_chunk,
system.cpp:177-370) through the C ABI.

Integer work, so every check is bit-exact:
  * the encoder ids the device builds from its context equal the oracle's
    build_encoder_inputs_host (system.cpp:62-95), with and without a style,
    with empty (-1) slots, before and after a roll;
  * the RVQ codes equal the oracle's llm_to_rvq (rvq.cpp:112-132) of the
    chunk's LLM ids, and the context equals the oracle's roll
    (system.cpp:315-333);
  * the chunk ids equal those of the host-side StreamingSession (context on
    the host, encoder ids uploaded each chunk), with and without the
    pipelined encoder (system.cpp:218-232, 334-370), also when the style
    changes between chunks;
  * an id at the wrong level fails as the reference's safe mode does and
    leaves the context and chunk index unchanged.
Tiny seeded model (d_model 128, codebook 8, 10-frame context, 4-frame chunks)
and the benchmark dims (1024-code levels, 250-frame context, 50-frame chunks).
"""

from __future__ import annotations


import numpy as np
import pytest

from oracle import system_oracle as so

pytestmark = pytest.mark.gpu

TINY_C = 8


@pytest.fixture(scope="module")
def tiny(gpu_available):
    import mrt_df
    import synth_bundle
    import system

    cfg = mrt_df.Config.tiny(TINY_C)
    w = synth_bundle.make_weights(cfg, seed=11, norm_jitter=0.1)
    scfg = system.SystemConfig(chunk_frames=4, context_frames=10, codebook_size=TINY_C)
    assert scfg.encoder_length == cfg.max_encoder_length
    ocfg = so.SystemConfig(codec_rvq_codebook_size=TINY_C, llm_vocab_size=cfg.vocab_size)
    model = mrt_df.Depthformer(w, cfg, dtype="bf16")
    rng = np.random.default_rng(7)
    style_lo = 2 + 16 * TINY_C
    style_a = (style_lo + TINY_C * np.arange(6) + rng.integers(0, TINY_C, 6)).astype(np.int32)
    style_b = (style_lo + TINY_C * np.arange(6) + rng.integers(0, TINY_C, 6)).astype(np.int32)
    assert style_a.max() < cfg.vocab_size and not np.array_equal(style_a, style_b)
    yield dict(mrt_df=mrt_df, system=system, cfg=cfg, scfg=scfg, ocfg=ocfg, model=model,
               style_a=style_a, style_b=style_b)
    model.close()


def _stream(env, **kw):
    mrt_df, scfg = env["mrt_df"], env["scfg"]
    return mrt_df.Stream(env["model"], mrt_df.StreamConfig(
        chunk_frames=scfg.chunk_frames, context_frames=scfg.context_frames, codebook_size=scfg.codebook_size,
        **kw))


def _chunk_opts(env, seed, pipeline=False, temperature=1.1, top_k=4):
    return env["mrt_df"].ChunkOptions(temperature=temperature, top_k=top_k, guidance_weight=5.0, seed=seed,
                                      pipeline_encoder=pipeline)


@pytest.mark.parametrize("pipeline", [False, True])
def test_stream_matches_oracle_plumbing(tiny, pipeline):
    mrt_df = tiny["mrt_df"]
    s = _stream(tiny)
    ctx0, idx0 = s.get_context()
    np.testing.assert_array_equal(ctx0, np.full((10, 16), -1, np.int32))  # empty_state
    assert idx0 == 0
    expect_ctx = ctx0
    styles = [tiny["style_a"], tiny["style_a"], None, tiny["style_b"], tiny["style_b"]]
    for i, style in enumerate(styles):
        llm, rvq = s.generate_chunk(style, _chunk_opts(tiny, seed=100 + i, pipeline=pipeline))
        if not pipeline:
            # the ids this chunk was encoded from: built from the pre-roll context
            enc = s.state.read(mrt_df.BUF_ENC_TOKENS).cpu().numpy()
            np.testing.assert_array_equal(enc, so.build_encoder_inputs_host(expect_ctx, tiny["ocfg"], style))
        np.testing.assert_array_equal(rvq, so.llm_to_rvq(llm, TINY_C, 2))
        expect_ctx = so.roll_context(expect_ctx, rvq)
        ctx, idx = s.get_context()
        np.testing.assert_array_equal(ctx, expect_ctx)
        assert idx == i + 1
        if pipeline:
            # the next chunk's ids, enqueued before returning: built from the rolled context
            enc = s.state.read(mrt_df.BUF_ENC_TOKENS).cpu().numpy()
            np.testing.assert_array_equal(enc, so.build_encoder_inputs_host(expect_ctx, tiny["ocfg"], style))
    s.close()


def test_stream_matches_host_session(tiny):
    system = tiny["system"]
    styles = [tiny["style_a"], tiny["style_a"], tiny["style_b"], None, None, tiny["style_a"]]
    host = system.StreamingSession(tiny["model"], tiny["scfg"], style=None, seed=31, top_k=4)
    ref_llm = []
    for st in styles:
        host.style = st
        host.generate_chunk()
        ref_llm.append(host.last_llm)
    for pipeline in (False, True):
        s = _stream(tiny)
        for i, st in enumerate(styles):
            llm, rvq = s.generate_chunk(st, _chunk_opts(tiny, seed=31 + i, pipeline=pipeline))
            np.testing.assert_array_equal(llm, ref_llm[i], err_msg=f"pipeline={pipeline} chunk {i}")
        np.testing.assert_array_equal(s.get_context()[0], host.context)
        s.close()
    host.state.close()


def test_stream_set_context_with_empty_slots(tiny):
    mrt_df = tiny["mrt_df"]
    rng = np.random.default_rng(3)
    ctx = rng.integers(0, TINY_C, size=(10, 16)).astype(np.int32)
    ctx[rng.random((10, 16)) < 0.3] = -1
    s = _stream(tiny)
    s.set_context(ctx, chunk_index=5)
    assert s.chunk_index == 5
    llm, rvq = s.generate_chunk(tiny["style_b"], _chunk_opts(tiny, seed=9))
    enc = s.state.read(mrt_df.BUF_ENC_TOKENS).cpu().numpy()
    np.testing.assert_array_equal(enc, so.build_encoder_inputs_host(ctx, tiny["ocfg"], tiny["style_b"]))
    np.testing.assert_array_equal(s.get_context()[0], so.roll_context(ctx, so.llm_to_rvq(llm, TINY_C, 2)))
    assert s.chunk_index == 6
    with pytest.raises(mrt_df.MrtError, match="code out of range"):
        bad = ctx.copy()
        bad[2, 3] = TINY_C
        s.set_context(bad)
    with pytest.raises(mrt_df.MrtError, match="style token out of range"):
        s.generate_chunk(np.full(6, tiny["cfg"].vocab_size, np.int32), _chunk_opts(tiny, seed=1))
    s.close()


@pytest.mark.parametrize("where,value", [((1, 3), 2 + TINY_C * 2 + 1),   # level 2's id at level 3
                                         ((3, 0), 0),                     # below the codec offset
                                         ((0, 15), 2 + TINY_C * 16)])     # past the last level
def test_stream_level_mismatch_raises(tiny, where, value):
    mrt_df = tiny["mrt_df"]
    s = _stream(tiny)
    good = (2 + TINY_C * np.arange(16)[None, :]
            + np.random.default_rng(1).integers(0, TINY_C, (4, 16))).astype(np.int32)
    s.generate_chunk(tiny["style_a"], _chunk_opts(tiny, seed=1), teacher=good)
    before, idx = s.get_context()
    teacher = good.copy()
    teacher[where] = value
    with pytest.raises(IndexError):
        so.llm_to_rvq(teacher, TINY_C, 2)  # the oracle rejects the same ids
    with pytest.raises(mrt_df.MrtError, match="token levels do not match expected RVQ structure") as e:
        s.generate_chunk(tiny["style_a"], _chunk_opts(tiny, seed=2, pipeline=True), teacher=teacher)
    assert e.value.code == 1
    after, idx2 = s.get_context()
    np.testing.assert_array_equal(after, before)
    assert idx2 == idx
    # the error flag is cleared: the next valid chunk goes through
    llm, rvq = s.generate_chunk(tiny["style_a"], _chunk_opts(tiny, seed=3), teacher=good)
    np.testing.assert_array_equal(llm, good)
    np.testing.assert_array_equal(rvq, so.llm_to_rvq(good, TINY_C, 2))
    s.close()


def test_stream_full_size_matches_host_session(gpu_available):
    """Benchmark dims: three 50-frame chunks over a 250-frame context, bf16."""
    import mrt_df
    import synth_bundle
    import system

    cfg = mrt_df.Config.bench()
    model = mrt_df.Depthformer(synth_bundle.make_weights(cfg, seed=1234, threads=16), cfg, dtype="bf16")
    scfg = system.SystemConfig()
    ocfg = so.SystemConfig()
    rng = np.random.default_rng(42)
    style = (scfg.style_offset + 1024 * np.arange(6) + rng.integers(0, 1024, 6)).astype(np.int32)
    host = system.StreamingSession(model, scfg, style=style, seed=77)
    dev = system.DeviceStreamingSession(model, scfg, style=style, seed=77, pipeline_encoder=True)
    expect_ctx = np.full((250, 16), -1, np.int32)
    for i in range(3):
        rvq_h = host.generate_chunk()
        rvq_d = dev.generate_chunk()
        if i == 0:
            enc = dev.state.read(mrt_df.BUF_ENC_TOKENS).cpu().numpy()
            # pipelined: the buffer already holds the next chunk's ids
            np.testing.assert_array_equal(
                enc, so.build_encoder_inputs_host(so.roll_context(expect_ctx, rvq_d), ocfg, style))
        np.testing.assert_array_equal(rvq_d, rvq_h, err_msg=f"chunk {i}")
        np.testing.assert_array_equal(rvq_d, so.llm_to_rvq(dev.last_llm, 1024, 2))
        expect_ctx = so.roll_context(expect_ctx, rvq_d)
        np.testing.assert_array_equal(dev.context, expect_ctx)
    assert dev.chunk_index == 3
    dev.stream.close()
    host.state.close()
    model.close()


@pytest.mark.parametrize("pipeline", [False, True])
def test_stream_audio_matches_oracle(tiny, pipeline):
    """The whole System::generate_chunk (system.cpp:177-440) on the device: the
    decoder input of each chunk is [the context frame before it (clamped; zeros
    on chunk 0), the chunk's codes] (bit-exact through the oracle's
    codec_input_frames), the codec output within 1e-4 of the oracle's fp32
    decode, the crossfade against the previous chunk's tail as the oracle's
    crossfade_chunk.  A token-only chunk in between drops the tail (no
    crossfade on the next audio chunk)."""
    import synth_bundle
    from oracle import codec_oracle as CO
    mrt_df = tiny["mrt_df"]
    shape = synth_bundle.CodecShape.tiny()
    w = synth_bundle.make_codec_weights(shape, levels=16, codebook=TINY_C)
    codec = mrt_df.Codec(w, max_frames=5, channels=shape.channels(), codebook_size=TINY_C)
    oc = CO.OracleCodec(w, CO.CodecConfig.tiny(), "fp32")
    s = _stream(tiny)
    s.attach_codec(codec)
    ctx = np.full((10, 16), -1, np.int32)
    ctx[3:6] = np.random.default_rng(3).integers(0, TINY_C, size=(3, 16))  # a mix of empty and set slots
    s.set_context(ctx, 0)
    tail = None
    plan = ["audio", "audio", "audio", "tokens", "audio"]
    for i, kind in enumerate(plan):
        before, idx = s.get_context()
        if kind == "tokens":
            s.generate_chunk(tiny["style_a"], _chunk_opts(tiny, seed=300 + i, pipeline=pipeline))
            tail = None
            continue
        llm, rvq, audio = s.generate_chunk_audio(tiny["style_a"], _chunk_opts(tiny, seed=300 + i, pipeline=pipeline))
        frames = so.codec_input_frames(before, rvq, idx)
        wave = oc.decode(frames)
        exp, tail = so.crossfade_chunk(wave, tail, idx)
        assert audio.shape == (4 * 1920, 2)
        err = float(np.linalg.norm(audio - exp) / np.linalg.norm(exp))
        print(f"chunk {i}: index {idx}, rel err {err:.2e}", flush=True)
        assert err <= 1e-4, (i, err)
        after, _ = s.get_context()
        np.testing.assert_array_equal(after, so.roll_context(before, rvq))
    s.attach_codec(None)
    with pytest.raises(mrt_df.MrtError):
        s.generate_chunk_audio(None, _chunk_opts(tiny, seed=9))
    big = mrt_df.Codec(w, max_frames=4, channels=shape.channels(), codebook_size=TINY_C)
    with pytest.raises(mrt_df.MrtError) as e:  # 4 frames + 1 crossfade frame do not fit
        s.attach_codec(big)
    assert "max_frames" in str(e.value)
    s.close()
    codec.close()
    big.close()


def test_stream_adaptive_speculation(tiny):
    """speculative = 2: a chunk speculates only its first 2 frames (a probe;
    the other frames take one frame launch each); when at least a quarter of
    the probed levels came from the verification pass, whole chunks
    speculate while that holds; after a miss, 4 chunks decode plainly before
    the next probe, 8 after a further miss, and so on.  The expected mode and
    launch count (a speculated frame: the temporal step and one launch of
    its open levels) of every chunk are replayed from the acceptance each
    speculating chunk reported, and the acceptance is taken over the
    speculated frames only."""
    mrt_df = tiny["mrt_df"]
    s = _stream(tiny)
    F, L, probe = 4, 16, 2
    pause, backoff, full, modes, accs = 0, 4, False, [], []
    for i in range(12):
        o = mrt_df.ChunkOptions(temperature=1.1, top_k=4, guidance_weight=5.0, speculative=2)  # seed: base + index
        s.generate_chunk(tiny["style_a"], o)
        launches = s.state.decode_time()[1]
        acc = s.state.spec_acceptance()
        modes.append(launches)
        accs.append(acc)
        # the policy, replayed: the first chunk has no drafts; a paused chunk decodes plainly
        spec = i > 0 and pause == 0
        # a speculated frame: the temporal step and one launch of its open levels
        want = (F * 2 if full else probe * 2 + (F - probe)) if spec else F
        assert launches == want, (i, modes, accs)
        assert (acc >= 0.0) == spec
        if spec and not full:
            # the probe's share comes from its 2 speculated frames: a multiple of 1 / 32
            assert abs(acc * probe * L - round(acc * probe * L)) < 1e-6
        if pause > 0:
            pause -= 1
        elif acc >= 0.25:
            full, backoff = True, 4
        elif acc >= 0.0:
            full, pause, backoff = False, backoff, min(2 * backoff, 64)
    print("launches", modes, "acceptance", [round(a, 3) for a in accs], flush=True)
    s.close()
