"""Codec decode on the GPU (system.cpp:373-390) against the oracle, through the
C ABI: RVQ dequantisation bit-exact; every decoder block output, the decoder's
spectrum, the windowed iSTFT frames and the audio within 1e-4 (norm-wise
relative, fp32 as the reference runs the codec); host and device entry points
identical; a second frame count on the same handle; id and size errors."""

from __future__ import annotations

import numpy as np
import pytest

import synth_bundle
from oracle import codec_oracle as C

pytestmark = pytest.mark.gpu

TOL = 1e-4


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _channels(cfg):
    return (cfg.embedding_dim, cfg.proj_ch, [b.in_ch for b in cfg.blocks], [b.out_ch for b in cfg.blocks])


def _check(codec, cfg, w, tok):
    import mrt_df
    S = tok.shape[0]
    print(f"codec decode: frames {S}, embedding {cfg.embedding_dim}", flush=True)
    audio = codec.decode(tok)
    rec = {}
    ref = C.OracleCodec(w, cfg, "fp32").decode(tok, rec)
    H = 4 * S
    Hn = S + 1
    emb = codec.read(mrt_df.CODEC_BUF_EMB, (Hn, cfg.embedding_dim))
    np.testing.assert_array_equal(emb[:S], rec["embeddings"])  # same level order, fp32 adds
    assert not emb[S].any()
    ic = codec.read(mrt_df.CODEC_BUF_INPUT_CONV, rec["input_conv"].shape)
    errs = {"input_conv": rel(ic, rec["input_conv"])}
    for i in range(7):
        b = codec.read(mrt_df.CODEC_BUF_BLOCK0 + i, rec[f"block{i}"].shape)
        errs[f"block{i}"] = rel(b, rec[f"block{i}"])
    spec = codec.read(mrt_df.CODEC_BUF_SPEC, (2, H, 480, 2))
    errs["spec"] = rel(spec, rec["spec_planar"])
    errs["audio"] = rel(audio, ref)
    print({k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    for k, v in errs.items():
        assert v <= TOL, (k, v)
    assert audio.shape == (S * 1920, 2)
    return audio


def test_codec_tiny_every_stage(gpu_available):
    import mrt_df
    cfg = C.CodecConfig.tiny()
    w = synth_bundle.make_codec_weights(synth_bundle.CodecShape.tiny(), levels=16, codebook=64)
    codec = mrt_df.Codec(w, max_frames=6, channels=_channels(cfg), codebook_size=64)
    rng = np.random.default_rng(0)
    _check(codec, cfg, w, rng.integers(0, 64, size=(5, 16)).astype(np.int32))
    # a smaller frame count on the same handle (its own launch plan)
    _check(codec, cfg, w, rng.integers(0, 64, size=(2, 16)).astype(np.int32))
    # one frame: the decoder's smallest input
    _check(codec, cfg, w, rng.integers(0, 64, size=(1, 16)).astype(np.int32))
    codec.close()


def test_codec_errors(gpu_available):
    import mrt_df
    cfg = C.CodecConfig.tiny()
    w = synth_bundle.make_codec_weights(synth_bundle.CodecShape.tiny(), levels=16, codebook=64)
    codec = mrt_df.Codec(w, max_frames=4, channels=_channels(cfg), codebook_size=64)
    tok = np.zeros((3, 16), np.int32)
    tok[1, 5] = 64
    with pytest.raises(mrt_df.MrtError) as e:
        codec.decode(tok)
    assert e.value.code == 1 and "token id" in str(e.value)
    tok[1, 5] = -1
    with pytest.raises(mrt_df.MrtError):
        codec.decode(tok)
    with pytest.raises(mrt_df.MrtError) as e:
        codec.decode(np.zeros((5, 16), np.int32))
    assert "max_frames" in str(e.value)
    assert np.isfinite(codec.decode(np.zeros((4, 16), np.int32))).all()
    codec.close()


@pytest.fixture(scope="module")
def full():
    import mrt_df
    cfg = C.CodecConfig.reference()
    w = synth_bundle.make_codec_weights(synth_bundle.CodecShape.reference())
    codec = mrt_df.Codec(w, max_frames=51)
    yield cfg, w, codec
    codec.close()


def test_codec_full_chunk(gpu_available, full):
    """One chunk at the reference's size: 1 crossfade frame + 50 frames."""
    cfg, w, codec = full
    tok = np.random.default_rng(1).integers(0, 1024, size=(51, 16)).astype(np.int32)
    _check(codec, cfg, w, tok)


def test_codec_device_entry_matches_host(gpu_available, full):
    import torch
    cfg, w, codec = full
    tok = np.random.default_rng(2).integers(0, 1024, size=(51, 16)).astype(np.int32)
    host = codec.decode(tok)
    td = torch.from_numpy(tok).cuda()
    ad = torch.empty((51 * 1920, 2), dtype=torch.float32, device="cuda")
    codec.decode_device(td, ad)
    codec.sync()
    np.testing.assert_array_equal(ad.cpu().numpy(), host)
    assert codec.decode_time() > 0
