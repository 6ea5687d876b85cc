"""C-ABI boundary checks that need no GPU.

The library must load and export every function include/mrt_df.h declares;
the config helpers must return the reference's DepthformerConfig values
(depthformer/model.cpp:34-48); and bundle / argument errors must come back
as status codes with a message (the reference throws std::runtime_error /
std::out_of_range at the same places: weights.cpp:129-130, model.cpp:216-218)
before any device call is made.
"""

from __future__ import annotations

import ctypes
import dataclasses
import json
import struct

import numpy as np
import pytest

import mrt_df
import synth_bundle

MRT_ERR_INVALID, MRT_ERR_HIP, MRT_ERR_MISSING_KEY, MRT_ERR_FORMAT = 1, 3, 4, 5


@pytest.fixture(scope="module")
def lib():
    return mrt_df.load_library()


def test_exports_every_header_function(lib):
    names = mrt_df.header_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_header_functions_all_have_signatures(lib):
    # every declared entry point is bound with explicit argtypes by the binding
    for n in mrt_df.header_functions():
        assert getattr(lib, n).argtypes is not None, n


def _cfg(lib, which):
    c = mrt_df._Config()
    getattr(lib, f"mrt_df_config_{which}")(ctypes.byref(c))
    return {f: getattr(c, f) for f in mrt_df.CONFIG_FIELDS}


def test_config_base_matches_reference(lib):
    # DepthformerConfig defaults (model.h:47-68) and base() (model.cpp:34-36)
    c = _cfg(lib, "base")
    assert c == dict(vocab_size=29824, d_model=768, d_kv=64, d_ff=2048, num_heads=12, num_encoder_layers=12,
                     num_temporal_layers=20, num_depth_layers=4, max_encoder_length=1006, rvq_depth=16,
                     temporal_num_buckets=128, temporal_max_distance=128, depth_num_buckets=16,
                     depth_max_distance=16)


def test_config_large_matches_reference(lib):
    # large() as the reference defines it (model.cpp:38-48)
    c = _cfg(lib, "large")
    assert (c["d_model"], c["num_heads"], c["d_ff"]) == (1024, 16, 2816)
    assert (c["num_encoder_layers"], c["num_temporal_layers"], c["num_depth_layers"]) == (24, 40, 8)
    assert c["vocab_size"] == 29824 and c["rvq_depth"] == 16


def test_error_message_is_per_call(lib):
    c = mrt_df._Config()
    code = lib.mrt_df_get_config(None, ctypes.byref(c), None)
    assert code == MRT_ERR_INVALID and b"null" in lib.mrt_last_error()


def _create_path(lib, path, cfg=None, dtype=mrt_df.DTYPE_BF16):
    c = cfg.to_c() if cfg is not None else mrt_df.Config.tiny().to_c()
    h = ctypes.c_void_p()
    code = lib.mrt_df_create(str(path).encode(), ctypes.byref(c), dtype, 0, ctypes.byref(h))
    return code, lib.mrt_last_error().decode(), h


def test_missing_bundle_file(lib, tmp_path):
    code, msg, h = _create_path(lib, tmp_path / "nope.safetensors")
    assert code == MRT_ERR_MISSING_KEY and "not a file" in msg and not h.value


def test_malformed_bundle(lib, tmp_path):
    p = tmp_path / "bad.safetensors"
    p.write_bytes(b"\x05\x00\x00\x00\x00\x00\x00\x00{oops")
    code, msg, h = _create_path(lib, p)
    assert code == MRT_ERR_FORMAT and not h.value, msg


def test_bundle_offsets_out_of_range(lib, tmp_path):
    hdr = json.dumps({"w": {"dtype": "F32", "shape": [4], "data_offsets": [0, 64]}}).encode()
    p = tmp_path / "short.safetensors"
    p.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\x00" * 16)
    code, msg, _ = _create_path(lib, p)
    assert code == MRT_ERR_FORMAT and "out of range" in msg


def _raw_bundle(tmp_path, entries, data_len=16, name="raw.safetensors"):
    hdr = json.dumps(entries).encode()
    p = tmp_path / name
    p.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\x00" * data_len)
    return p


@pytest.mark.parametrize("shape,why", [
    ([2 ** 44, 1024, 256], "bad dimension"),        # beyond 2^40 along one axis
    ([2 ** 40, 2 ** 40, 2 ** 40], "overflows"),     # each axis allowed, the product wraps 64 bits
    ([-4], "bad dimension"),
    ([2.5], "bad dimension"),
    (["4"], "bad dimension"),
])
def test_bundle_rejects_bad_shapes(lib, tmp_path, shape, why):
    """A header shape must be non-negative integers whose element count and byte
    size do not overflow, and the bytes must equal the data_offsets span: a
    codebook entry of shape [2^44, 1024, 256] over 0 bytes is refused before any
    reader trusts its size."""
    p = _raw_bundle(tmp_path, {"codebooks": {"dtype": "F32", "shape": shape, "data_offsets": [0, 0]}})
    code, msg, h = _create_path(lib, p)
    assert code == MRT_ERR_FORMAT and why in msg and not h.value, msg


def test_bundle_size_must_equal_offsets_span(lib, tmp_path):
    p = _raw_bundle(tmp_path, {"w": {"dtype": "F32", "shape": [2], "data_offsets": [0, 16]}})
    code, msg, _ = _create_path(lib, p)
    assert code == MRT_ERR_FORMAT and "size mismatch" in msg
    p = _raw_bundle(tmp_path, {"w": {"dtype": "BF16", "shape": [4], "data_offsets": [0, 16]}}, name="b.safetensors")
    code, msg, _ = _create_path(lib, p)
    assert code == MRT_ERR_FORMAT and "size mismatch" in msg
    p = _raw_bundle(tmp_path, {"w": {"dtype": "F32", "shape": [1], "data_offsets": [-4, 0]}}, name="n.safetensors")
    code, msg, _ = _create_path(lib, p)
    assert code == MRT_ERR_FORMAT and "out of range" in msg


def test_codec_codebooks_with_huge_shape_are_refused(lib, tmp_path):
    """The codec's codebooks file goes through the same reader: a (2^44, 1024,
    256) codebook over no bytes is refused while the files are read."""
    dec = _raw_bundle(tmp_path, {"w": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}, name="dec.safetensors")
    cbs = _raw_bundle(tmp_path, {"codebooks": {"dtype": "F32", "shape": [2 ** 44, 1024, 256], "data_offsets": [0, 0]}},
                      name="cb.safetensors")
    c = mrt_df._CodecConfig()
    lib.mrt_codec_config_default(ctypes.byref(c))
    h = ctypes.c_void_p()
    code = lib.mrt_codec_create(str(dec).encode(), str(cbs).encode(), ctypes.byref(c), 0, ctypes.byref(h))
    msg = lib.mrt_last_error().decode()
    assert code == MRT_ERR_FORMAT and "bad dimension" in msg and not h.value, msg


def test_bundle_missing_key(lib, tmp_path):
    cfg = mrt_df.Config.tiny()
    w = synth_bundle.make_weights(cfg, seed=1)
    w.pop("decoder_norm.weight")
    p = tmp_path / "partial.safetensors"
    synth_bundle.write_bundle(p, w)
    code, msg, _ = _create_path(lib, p, cfg)
    assert code == MRT_ERR_MISSING_KEY and "decoder_norm.weight" in msg


def test_bundle_shape_mismatch(lib, tmp_path):
    cfg = mrt_df.Config.tiny()
    w = synth_bundle.make_weights(cfg, seed=1)
    w["lm_head.weight"] = w["lm_head.weight"][:-1]
    p = tmp_path / "shape.safetensors"
    synth_bundle.write_bundle(p, w)
    code, msg, _ = _create_path(lib, p, cfg)
    assert code == MRT_ERR_INVALID and "lm_head.weight" in msg


def test_unsupported_head_dim(lib, tmp_path):
    cfg = mrt_df.Config.tiny()
    bad = dataclasses.replace(cfg, d_kv=32)
    p = tmp_path / "any.safetensors"
    synth_bundle.write_bundle(p, synth_bundle.make_weights(cfg, seed=1))
    code, msg, _ = _create_path(lib, p, bad)
    assert code == MRT_ERR_INVALID and "d_kv" in msg


def test_unknown_dtype(lib, tmp_path):
    cfg = mrt_df.Config.tiny()
    p = tmp_path / "ok.safetensors"
    synth_bundle.write_bundle(p, synth_bundle.make_weights(cfg, seed=1))
    code, msg, _ = _create_path(lib, p, cfg, dtype=7)
    assert code == MRT_ERR_INVALID and "dtype" in msg


def test_parse_dtype_spellings():
    """The dtype flag (dtype.cpp:35-56), cases of the reference's
    tests/test_dtype.cpp:24-50: every spelling, case-insensitive, maps to its
    ABI code; nonsense raises; names round-trip."""
    for name in ("fp32", "float32", "F32", "f32"):
        assert mrt_df.dtype_code(name) == mrt_df.DTYPE_F32
    for name in ("fp16", "float16", "Half", "f16"):
        assert mrt_df.dtype_code(name) == mrt_df.DTYPE_F16
    for name in ("bf16", "bfloat16", "BF16"):
        assert mrt_df.dtype_code(name) == mrt_df.DTYPE_BF16
    for bad in ("int8", "", "bf32"):
        with pytest.raises(ValueError, match="expected fp32\\|fp16\\|bf16"):
            mrt_df.parse_dtype(bad)
    for name in ("fp32", "fp16", "bf16"):
        assert mrt_df.dtype_name(mrt_df.dtype_code(name)) == name
    assert mrt_df.dtype_name(7) == "unsupported"


def test_fp16_code_passes_the_dtype_check(lib, tmp_path):
    """MRT_DTYPE_F16 is accepted by mrt_df_create (the error, if any, comes
    from the device, not the dtype check)."""
    cfg = mrt_df.Config.tiny()
    p = tmp_path / "ok.safetensors"
    synth_bundle.write_bundle(p, synth_bundle.make_weights(cfg, seed=1))
    code, msg, h = _create_path(lib, p, cfg, dtype=mrt_df.DTYPE_F16)
    assert code in (0, MRT_ERR_HIP), msg
    if code == 0:
        lib.mrt_df_destroy(h)


def test_valid_bundle_reaches_the_device(lib, tmp_path):
    """A complete bundle passes every host check; without a GPU the first
    device call fails with MRT_ERR_HIP, with one it loads."""
    cfg = mrt_df.Config.tiny()
    p = tmp_path / "tiny.safetensors"
    synth_bundle.write_bundle(p, synth_bundle.make_weights(cfg, seed=1))
    code, msg, h = _create_path(lib, p, cfg)
    assert code in (0, MRT_ERR_HIP), msg
    if code == 0:
        lib.mrt_df_destroy(h)


def test_null_arguments(lib):
    c = mrt_df.Config.tiny().to_c()
    h = ctypes.c_void_p()
    assert lib.mrt_df_create(None, ctypes.byref(c), 1, 0, ctypes.byref(h)) == MRT_ERR_INVALID
    assert lib.mrt_df_state_create(None, 2, 4, 8, ctypes.byref(h)) == MRT_ERR_INVALID
    assert lib.mrt_df_sync(None) == MRT_ERR_INVALID
    assert lib.mrt_df_encode(None, None) == MRT_ERR_INVALID
    assert lib.mrt_df_depth_step(None, None, 0, 0, 8, 2, None) == MRT_ERR_INVALID
    assert lib.mrt_df_temporal_step(None, None, None, 0, None) == MRT_ERR_INVALID
    assert lib.mrt_df_generate_tokens(None, None, None, None) == MRT_ERR_INVALID
    sz = ctypes.c_size_t()
    assert lib.mrt_df_state_buffer_bytes(None, 0, ctypes.byref(sz)) == MRT_ERR_INVALID
    assert lib.mrt_df_state_set_cache_length(None, 0, 0) == MRT_ERR_INVALID


def test_create_from_tensors_rejects_bad_entries(lib):
    cfg = mrt_df.Config.tiny().to_c()
    h = ctypes.c_void_p()
    names = (ctypes.c_char_p * 1)(None)
    data = (ctypes.c_void_p * 1)(None)
    shapes = (ctypes.c_void_p * 1)(None)
    ndims = (ctypes.c_int32 * 1)(1)
    code = lib.mrt_df_create_from_tensors(1, names, data, shapes, ndims, ctypes.byref(cfg), 1, 0,
                                          ctypes.byref(h))
    assert code == MRT_ERR_INVALID and b"bad tensor entry" in lib.mrt_last_error()


def test_bundle_layout_matches_reference_keys():
    """Key set of the bundle layout (model.cpp:177-198, modules.cpp:342-381) at the tiny dims."""
    cfg = mrt_df.Config.tiny()
    layout = dict(synth_bundle.bundle_layout(cfg))
    keys = set(layout)
    assert {"token_embedding.weight", "lm_head.weight", "encoder_norm.weight", "decoder_norm.weight",
            "temporal_rel_pos.relative_attention_bias.weight",
            "depth_rel_pos.relative_attention_bias.weight"} <= keys
    for i in range(cfg.num_temporal_layers):
        for k in ("pre_self_attn_norm", "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                  "self_attn.o_proj", "pre_cross_attn_norm", "cross_attn.q_proj", "cross_attn.k_proj",
                  "cross_attn.v_proj", "cross_attn.o_proj", "pre_ffn_norm", "ffn.wi_0", "ffn.wi_1", "ffn.wo"):
            assert f"temporal_layers.{i}.{k}.weight" in keys
    for i in range(cfg.num_depth_layers):
        assert f"depth_layers.{i}.pre_self_attn_norm.weight" in keys
        assert f"depth_layers.{i}.cross_attn.q_proj.weight" not in keys
    assert tuple(layout["lm_head.weight"]) == (cfg.vocab_size, cfg.d_model)
    assert tuple(layout["temporal_layers.0.ffn.wo.weight"]) == (cfg.d_model, cfg.d_ff)
    assert np.prod(layout["temporal_rel_pos.relative_attention_bias.weight"]) == \
        cfg.temporal_num_buckets * cfg.num_heads
