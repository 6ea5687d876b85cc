"""Codec C-ABI checks that need no GPU: the default configuration is the
reference's decoder (spectrostream.cpp:328-362, SystemConfig's 1 crossfade
frame + 50 chunk frames) and bundle errors come back as status codes before
any device call (WeightBundle::tensor throws std::out_of_range for a missing
key, weights.cpp:126-133)."""

from __future__ import annotations

import ctypes

import pytest

import mrt_df
import synth_bundle

MRT_ERR_INVALID, MRT_ERR_MISSING_KEY = 1, 4


@pytest.fixture(scope="module")
def tiny_weights():
    shape = synth_bundle.CodecShape.tiny()
    return shape, synth_bundle.make_codec_weights(shape, levels=16, codebook=64)


def _channels(shape):
    return shape.channels()


def test_codec_config_default_is_the_reference_decoder():
    lib = mrt_df.load_library()
    c = mrt_df._CodecConfig()
    lib.mrt_codec_config_default(ctypes.byref(c))
    ref = synth_bundle.CodecShape.reference()
    assert (c.embedding_dim, c.proj_channels, c.unfold) == (256, 2560, 5)
    assert list(c.block_in) == [b.in_ch for b in ref.blocks]
    assert list(c.block_out) == [b.out_ch for b in ref.blocks]
    assert (c.rvq_levels, c.codebook_size, c.max_frames) == (16, 1024, 51)


def test_codec_missing_key(tiny_weights):
    cfg, w = tiny_weights
    w = dict(w)
    del w["decoder_blocks.4.shortcut.bias"]
    with pytest.raises(mrt_df.MrtError) as e:
        mrt_df.Codec(w, max_frames=4, channels=_channels(cfg), codebook_size=64)
    assert e.value.code == MRT_ERR_MISSING_KEY and "decoder_blocks.4.shortcut.bias" in str(e.value)


def test_codec_shape_mismatch(tiny_weights):
    cfg, w = tiny_weights
    w = dict(w)
    w["decoder_blocks.2.conv_transpose.weight"] = w["decoder_blocks.2.conv_transpose.weight"][:, :, :, :3].copy()
    with pytest.raises(mrt_df.MrtError) as e:
        mrt_df.Codec(w, max_frames=4, channels=_channels(cfg), codebook_size=64)
    assert e.value.code == MRT_ERR_INVALID and "conv_transpose.weight" in str(e.value)


def test_codec_bad_codebooks(tiny_weights):
    cfg, w = tiny_weights
    with pytest.raises(mrt_df.MrtError) as e:
        mrt_df.Codec(w, max_frames=4, channels=_channels(cfg), codebook_size=1024)  # tensor has 64 codes
    assert e.value.code == MRT_ERR_INVALID and "codebooks" in str(e.value)


def test_codec_bad_channel_chain(tiny_weights):
    cfg, w = tiny_weights
    e_, p_, bi, bo = _channels(cfg)
    bi = list(bi)
    bi[3] = bi[3] * 2
    with pytest.raises(mrt_df.MrtError) as e:
        mrt_df.Codec(w, max_frames=4, channels=(e_, p_, bi, bo), codebook_size=64)
    assert e.value.code == MRT_ERR_INVALID
