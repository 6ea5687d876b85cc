"""MusicCoCa / StyleModel C-ABI checks that need no GPU: the default
configuration is the reference's (musiccoca.h:151-162, style_model.h:24-27)
and bundle errors come back as status codes before any device call."""

from __future__ import annotations

import ctypes

import pytest

import mrt_df
import synth_bundle

MRT_ERR_INVALID, MRT_ERR_MISSING_KEY = 1, 4


def test_coca_config_default_is_the_reference():
    lib = mrt_df.load_library()
    c = mrt_df._CocaConfig()
    lib.mrt_coca_config_default(ctypes.byref(c))
    got = {f: getattr(c, f) for f, _ in mrt_df._CocaConfig._fields_}
    assert got == dict(d_model=768, num_heads=12, d_head=64, d_ff=3072, num_layers=12, pooler_d_head=256,
                       vocab_size=64000, max_text_len=128, rvq_depth=12, codebook_size=1024)


@pytest.fixture(scope="module")
def tiny():
    cfg = mrt_df.CocaConfig.tiny()
    return cfg, synth_bundle.make_coca_weights(cfg)


def test_coca_missing_key(tiny):
    cfg, w = tiny
    w = dict(w)
    del w["text_layers.1.ffn_w2.bias"]
    with pytest.raises(mrt_df.MrtError) as e:
        mrt_df.StyleModel(w, cfg)
    assert e.value.code == MRT_ERR_MISSING_KEY and "text_layers.1.ffn_w2.bias" in str(e.value)


def test_coca_shape_and_codebook_errors(tiny):
    cfg, w = tiny
    bad = dict(w)
    bad["text_pooler.attn._per_dim_scale"] = w["text_pooler.attn._per_dim_scale"][:5].copy()
    with pytest.raises(mrt_df.MrtError) as e:
        mrt_df.StyleModel(bad, cfg)
    assert e.value.code == MRT_ERR_INVALID and "_per_dim_scale" in str(e.value)
    bad = dict(w)
    bad["codebooks"] = w["codebooks"][:3].copy()  # fewer than rvq_depth levels
    with pytest.raises(mrt_df.MrtError) as e:
        mrt_df.StyleModel(bad, cfg)
    assert "codebooks" in str(e.value)


def test_coca_layout_matches_oracle_config():
    from oracle import musiccoca_oracle as M
    a, b = mrt_df.CocaConfig(), M.CocaConfig()
    assert {f: getattr(a, f) for f in vars(b)} == vars(b)
    t, u = mrt_df.CocaConfig.tiny(), M.CocaConfig.tiny()
    assert {f: getattr(t, f) for f in vars(u)} == vars(u)
