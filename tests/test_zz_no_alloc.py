"""mrt_df_sample_level_noalloc, the draw for callers that cannot allocate,
through the C ABI: its token equals mrt_df_sample_level's (the state-owned
draw sharing the same kernel) on two calls in a row, the second with a smaller
input, in both dtypes; calls enqueued on two streams at once each draw the
token of their own slice and seed (the seed travels by value; only the
discarded feedback rows share the scratch); a d_model whose feedback rows
exceed the fixed scratch is rejected before anything is enqueued."""

from __future__ import annotations

import ctypes
import dataclasses

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _noalloc(lib, mrt_df, model, slice_t, opts, frame, level, tok_t):
    o = mrt_df.State._opts(opts)
    return lib.mrt_df_sample_level_noalloc(model._h, ctypes.c_void_p(slice_t.data_ptr()), ctypes.byref(o), frame,
                                           level, ctypes.c_void_p(tok_t.data_ptr()), None)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_noalloc_draw_equals_state_draw(gpu_available, dtype):
    import torch

    import mrt_df
    import synth_bundle

    lib = mrt_df.load_library()
    cfg = dataclasses.replace(mrt_df.Config.tiny(), vocab_size=2 + 22 * 1024)
    m = mrt_df.Depthformer(synth_bundle.make_weights(cfg, seed=3), cfg, dtype=dtype)
    st = m.new_state(max_frames=2)
    rng = np.random.default_rng(17)
    # the second call has a smaller slice (300 codes) and another frame / level
    for C, k, T, frame, level in [(1024, 40, 1.1, 3, 5), (300, 4, 0.7, 1, 2), (1024, 1, 40.0, 7, 15)]:
        sl = torch.tensor((rng.standard_normal((2, C)) * 3).astype(np.float32), device="cuda")
        opts = mrt_df.GenOptions(num_frames=2, rvq_depth=16, temperature=T, top_k=k, guidance_weight=5.0,
                                 seed=int(rng.integers(1 << 40)), codebook_size=C, codec_offset=2)
        exp = st.sample_level(sl, opts, frame=frame, level=level)
        tok = torch.full((1,), -1, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        code = _noalloc(lib, mrt_df, m, sl, opts, frame, level, tok)
        assert code == 0, lib.mrt_last_error().decode()
        torch.cuda.synchronize()
        assert int(tok.item()) == exp, (C, k, T, int(tok.item()), exp)
    st.close()
    m.close()


def test_noalloc_calls_on_two_streams_draw_their_own_tokens(gpu_available):
    import torch

    import mrt_df
    import synth_bundle

    lib = mrt_df.load_library()
    cfg = dataclasses.replace(mrt_df.Config.tiny(), vocab_size=2 + 22 * 1024)
    m = mrt_df.Depthformer(synth_bundle.make_weights(cfg, seed=3), cfg, dtype="bf16")
    st = m.new_state(max_frames=2)
    rng = np.random.default_rng(23)
    n = 24
    C = 1024
    slices = [torch.tensor((rng.standard_normal((2, C)) * 3).astype(np.float32), device="cuda") for _ in range(n)]
    optss = [mrt_df.GenOptions(num_frames=2, rvq_depth=16, temperature=1.1, top_k=40, guidance_weight=5.0,
                               seed=int(rng.integers(1 << 40)), codebook_size=C, codec_offset=2) for _ in range(n)]
    exp = [st.sample_level(slices[i], optss[i], frame=i % 5, level=i % 16) for i in range(n)]
    toks = torch.full((n,), -1, dtype=torch.int32, device="cuda")
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for i in range(n):  # alternate the streams, so consecutive calls overlap on the device
        o = mrt_df.State._opts(optss[i])
        code = lib.mrt_df_sample_level_noalloc(m._h, ctypes.c_void_p(slices[i].data_ptr()), ctypes.byref(o), i % 5,
                                               i % 16, ctypes.c_void_p(toks.data_ptr() + 4 * i),
                                               ctypes.c_void_p(streams[i % 2].cuda_stream))
        assert code == 0, lib.mrt_last_error().decode()
    torch.cuda.synchronize()
    assert toks.cpu().tolist() == exp
    st.close()
    m.close()


def test_noalloc_rejects_rows_beyond_the_scratch(gpu_available):
    import torch

    import mrt_df
    import synth_bundle

    lib = mrt_df.load_library()
    cfg = dataclasses.replace(mrt_df.Config.tiny(), d_model=1536)  # fp32: 6 x 1536 x 4 + 256 > 32 KiB
    m = mrt_df.Depthformer(synth_bundle.make_weights(cfg, seed=3), cfg, dtype="fp32")
    sl = torch.zeros((2, 8), dtype=torch.float32, device="cuda")
    tok = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    opts = mrt_df.GenOptions(num_frames=1, rvq_depth=16, codebook_size=8, codec_offset=2)
    torch.cuda.synchronize()
    code = _noalloc(lib, mrt_df, m, sl, opts, 0, 0, tok)
    assert code == 1 and "scratch" in lib.mrt_last_error().decode()
    torch.cuda.synchronize()
    assert int(tok.item()) == -1  # nothing was enqueued
    m.close()
