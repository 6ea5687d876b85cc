"""Python binding of ``libmrt_df.so`` (include/mrt_df.h) over ctypes.

Mirrors the reference's ``Depthformer`` surface (depthformer/model.h:72-239):
``encode``, ``temporal_step``, ``depth_step``, ``generate_tokens`` and
``sample_level`` (decode.cpp:124-148).  Device buffers are torch tensors
(torch is only the allocator here); all compute runs in the HIP library.
The library must be built (``build.py``); loading fails loudly otherwise.
"""

from __future__ import annotations

import ctypes
import dataclasses
import os
import pathlib
import re
from typing import Dict, Optional, Sequence

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "libmrt_df.so"
HEADER = HERE.parent / "include" / "mrt_df.h"

MRT_OK = 0
DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2


def parse_dtype(name: str) -> str:
    """``parse_dtype`` (dtype.cpp:35-49): case-insensitive fp32 | fp16 | bf16 and
    their aliases -> the canonical name; anything else raises ValueError."""
    n = str(name).lower()
    if n in ("fp32", "float32", "f32"):
        return "fp32"
    if n in ("fp16", "float16", "f16", "half"):
        return "fp16"
    if n in ("bf16", "bfloat16"):
        return "bf16"
    raise ValueError(f'unknown dtype "{name}"; expected fp32|fp16|bf16')


_DTYPE_CODE = {"fp32": DTYPE_F32, "bf16": DTYPE_BF16, "fp16": DTYPE_F16}


def dtype_code(name: str) -> int:
    """The ABI's MRT_DTYPE_* code of a dtype name (any alias parse_dtype accepts)."""
    return _DTYPE_CODE[parse_dtype(name)]


def dtype_name(code: int) -> str:
    """``dtype_name`` (dtype.cpp:51-56) of an ABI dtype code; "unsupported" otherwise."""
    return {v: k for k, v in _DTYPE_CODE.items()}.get(code, "unsupported")
BUF_ENC_OUT, BUF_CROSS_K, BUF_CROSS_V = 0, 1, 2
BUF_TEMPORAL_K, BUF_TEMPORAL_V, BUF_DEPTH_K, BUF_DEPTH_V = 3, 4, 5, 6
BUF_ENC_TOKENS = 7

CONFIG_FIELDS = ("vocab_size", "d_model", "d_kv", "d_ff", "num_heads", "num_encoder_layers",
                 "num_temporal_layers", "num_depth_layers", "max_encoder_length", "rvq_depth",
                 "temporal_num_buckets", "temporal_max_distance", "depth_num_buckets",
                 "depth_max_distance")


class MrtError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[mrt_df error {code}] {msg}")
        self.code = code


class _Config(ctypes.Structure):
    _fields_ = [(f, ctypes.c_int32) for f in CONFIG_FIELDS]


class _GenOpts(ctypes.Structure):
    _fields_ = [
        ("num_frames", ctypes.c_int32),
        ("rvq_depth", ctypes.c_int32),
        ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_int32),
        ("guidance_weight", ctypes.c_float),
        ("seed", ctypes.c_uint64),
        ("codebook_size", ctypes.c_int32),
        ("codec_offset", ctypes.c_int32),
        ("teacher", ctypes.POINTER(ctypes.c_int32)),
        ("use_graph", ctypes.c_int32),
        ("record_slices", ctypes.c_void_p),
        ("record_temporal", ctypes.c_void_p),
        ("record_drawn", ctypes.c_void_p),
        ("record_frame_mean", ctypes.c_void_p),
        ("speculative", ctypes.c_int32),
    ]


class _DecodeProfile(ctypes.Structure):
    _fields_ = [(n, ctypes.c_float) for n in ("total_ms", "encoder_ms", "bias_ms", "temporal_ms", "depth_ms",
                                               "sample_ms")] + [("frames", ctypes.c_int32)]


class _StreamConfig(ctypes.Structure):
    _fields_ = [(f, ctypes.c_int32) for f in (
        "chunk_frames", "context_frames", "codebook_size", "encoder_codec_rvq_depth",
        "encoder_style_rvq_depth", "decoder_codec_rvq_depth", "mask_token", "codec_offset",
        "crossfade_frames", "samples_per_frame")]


class _ChunkOpts(ctypes.Structure):
    _fields_ = [
        ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_int32),
        ("guidance_weight", ctypes.c_float),
        ("has_seed", ctypes.c_int32),
        ("seed", ctypes.c_uint64),
        ("pipeline_encoder", ctypes.c_int32),
        ("use_graph", ctypes.c_int32),
        ("teacher", ctypes.POINTER(ctypes.c_int32)),
        ("speculative", ctypes.c_int32),
    ]


class _CodecConfig(ctypes.Structure):
    _fields_ = [
        ("embedding_dim", ctypes.c_int32),
        ("proj_channels", ctypes.c_int32),
        ("unfold", ctypes.c_int32),
        ("block_in", ctypes.c_int32 * 7),
        ("block_out", ctypes.c_int32 * 7),
        ("rvq_levels", ctypes.c_int32),
        ("codebook_size", ctypes.c_int32),
        ("max_frames", ctypes.c_int32),
    ]


class _CocaConfig(ctypes.Structure):
    _fields_ = [(f, ctypes.c_int32) for f in (
        "d_model", "num_heads", "d_head", "d_ff", "num_layers", "pooler_d_head", "vocab_size", "max_text_len",
        "rvq_depth", "codebook_size")]


CODEC_BUF_EMB, CODEC_BUF_INPUT_CONV, CODEC_BUF_BLOCK0, CODEC_BUF_SPEC, CODEC_BUF_FRAMES = 0, 1, 2, 9, 10
COCA_BUF_EMBEDDING = 0


@dataclasses.dataclass(frozen=True)
class Config:
    """DepthformerConfig (model.h:47-68)."""

    vocab_size: int = 29824
    d_model: int = 768
    d_kv: int = 64
    d_ff: int = 2048
    num_heads: int = 12
    num_encoder_layers: int = 12
    num_temporal_layers: int = 20
    num_depth_layers: int = 4
    max_encoder_length: int = 1006
    rvq_depth: int = 16
    temporal_num_buckets: int = 128
    temporal_max_distance: int = 128
    depth_num_buckets: int = 16
    depth_max_distance: int = 16

    @staticmethod
    def base() -> "Config":
        return Config()

    @staticmethod
    def large() -> "Config":
        return Config(d_model=1024, d_kv=64, d_ff=2816, num_heads=16, num_encoder_layers=24,
                      num_temporal_layers=40, num_depth_layers=8)

    @staticmethod
    def bench() -> "Config":
        """d_model 1024, 16 heads x 64, d_ff 2816, 12/20/4 layers, vocab 29824."""
        return Config(d_model=1024, d_kv=64, d_ff=2816, num_heads=16, num_encoder_layers=12,
                      num_temporal_layers=20, num_depth_layers=4)

    @staticmethod
    def tiny(codebook: int = 8) -> "Config":
        return Config(vocab_size=2 + 22 * codebook, d_model=128, d_kv=64, d_ff=192, num_heads=2,
                      num_encoder_layers=2, num_temporal_layers=2, num_depth_layers=2,
                      max_encoder_length=46)

    def to_c(self) -> _Config:
        return _Config(*[getattr(self, f) for f in CONFIG_FIELDS])


@dataclasses.dataclass
class GenOptions:
    """GenerateOptions (decode.h:48-57) + vocab layout (system.h:44-83)."""

    num_frames: int = 50
    rvq_depth: int = 16
    temperature: float = 1.1
    top_k: int = 40
    guidance_weight: float = 5.0
    seed: int = 0
    codebook_size: int = 1024
    codec_offset: int = 2
    use_graph: bool = True
    speculative: bool = False


_lib = None


def read_bandwidth(nbytes: int, passes: int, device: int = 0) -> float:
    """Device read bandwidth in GB/s of `passes` reads of an `nbytes` buffer
    after one warm pass (mrt_probe_read_bandwidth)."""
    lib = load_library()
    out = ctypes.c_float()
    _check(lib, lib.mrt_probe_read_bandwidth(device, nbytes, passes, ctypes.byref(out)))
    return float(out.value)


def handoff_latency(workgroups: int, words: int, rounds: int, delay: int = 0, device: int = 0) -> float:
    """Microseconds per round of an all-gather of ``words`` tagged words among
    ``workgroups`` workgroups, the hand-off of one persistent-kernel phase,
    with ``delay`` rounds of s_sleep(1) before each first poll
    (mrt_probe_handoff)."""
    lib = load_library()
    out = ctypes.c_float()
    _check(lib, lib.mrt_probe_handoff(device, workgroups, words, rounds, delay, ctypes.byref(out)))
    return float(out.value)


def pingpong_latency(peer: int, rounds: int, device: int = 0) -> float:
    """One-way microseconds of a word bounced between workgroups 0 and ``peer``
    (mrt_probe_pingpong)."""
    lib = load_library()
    out = ctypes.c_float()
    _check(lib, lib.mrt_probe_pingpong(device, peer, rounds, ctypes.byref(out)))
    return float(out.value)


def header_functions(path: pathlib.Path = HEADER) -> list:
    """Names of the functions include/mrt_df.h declares."""
    text = re.sub(r"/\*.*?\*/", "", path.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mrt_[a-z0-9_]+)\s*\(", text)))


def load_library(path: Optional[os.PathLike] = None) -> ctypes.CDLL:
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = pathlib.Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"{p} is missing: build it with `python {HERE / 'build.py'}` "
                           "(there is no CPU fallback)")
    lib = ctypes.CDLL(str(p))
    vp, i32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    sig = {
        "mrt_last_error": (ctypes.c_char_p, []),
        "mrt_df_config_base": (None, [ctypes.POINTER(_Config)]),
        "mrt_df_config_large": (None, [ctypes.POINTER(_Config)]),
        "mrt_df_create": (i32, [ctypes.c_char_p, ctypes.POINTER(_Config), i32, i32, ctypes.POINTER(vp)]),
        "mrt_probe_read_bandwidth": (i32, [i32, sz, i32, ctypes.POINTER(ctypes.c_float)]),
        "mrt_probe_handoff": (i32, [i32, i32, i32, i32, i32, ctypes.POINTER(ctypes.c_float)]),
        "mrt_probe_pingpong": (i32, [i32, i32, i32, ctypes.POINTER(ctypes.c_float)]),
        "mrt_df_sample_level_noalloc": (i32, [vp, vp, ctypes.POINTER(_GenOpts), i32, i32, vp, vp]),
        "mrt_df_depth_forward_full": (i32, [vp, vp, i32, vp, i32, vp]),
        "mrt_df_temporal_step_with_bias": (i32, [vp, vp, vp, i32, vp, vp]),
        "mrt_df_depth_step_with_bias": (i32, [vp, vp, i32, vp, i32, i32, i32, vp]),
        "mrt_df_precompute_biases": (i32, [vp, i32, i32, vp]),
        "mrt_df_state_reset_cache": (i32, [vp, i32]),
        "mrt_df_create_from_tensors": (i32, [i32, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(vp),
                                             ctypes.POINTER(vp), ctypes.POINTER(ctypes.c_int32),
                                             ctypes.POINTER(_Config), i32, i32, ctypes.POINTER(vp)]),
        "mrt_df_destroy": (None, [vp]),
        "mrt_df_get_config": (i32, [vp, ctypes.POINTER(_Config), ctypes.POINTER(i32)]),
        "mrt_df_state_create": (i32, [vp, i32, i32, i32, ctypes.POINTER(vp)]),
        "mrt_df_state_destroy": (None, [vp]),
        "mrt_df_state_stream": (i32, [vp, ctypes.POINTER(vp)]),
        "mrt_df_sync": (i32, [vp]),
        "mrt_df_encode": (i32, [vp, ctypes.POINTER(ctypes.c_int32)]),
        "mrt_df_temporal_step": (i32, [vp, vp, vp, i32, vp]),
        "mrt_df_depth_step": (i32, [vp, vp, i32, i32, i32, i32, vp]),
        "mrt_df_generate_tokens": (i32, [vp, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(_GenOpts),
                                         ctypes.POINTER(ctypes.c_int32)]),
        "mrt_df_sample_level": (i32, [vp, vp, ctypes.POINTER(_GenOpts), i32, i32,
                                      ctypes.POINTER(ctypes.c_int32)]),
        "mrt_df_state_buffer_bytes": (i32, [vp, i32, ctypes.POINTER(sz)]),
        "mrt_df_state_read": (i32, [vp, i32, i32, vp, sz]),
        "mrt_df_state_write": (i32, [vp, i32, i32, vp, sz]),
        "mrt_df_state_set_cache_length": (i32, [vp, i32, i32]),
        "mrt_df_state_decode_time": (i32, [vp, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(i32)]),
        "mrt_df_state_phase_trace": (i32, [vp, ctypes.POINTER(ctypes.c_uint64), i32, ctypes.POINTER(ctypes.c_float)]),
        "mrt_df_state_spec_acceptance": (i32, [vp, ctypes.POINTER(ctypes.c_float)]),
        "mrt_df_state_set_profile": (i32, [vp, i32]),
        "mrt_df_state_decode_profile": (i32, [vp, ctypes.POINTER(_DecodeProfile)]),
        "mrt_df_state_compile": (i32, [vp, ctypes.POINTER(_GenOpts)]),
        "mrt_df_stream_compile": (i32, [vp, ctypes.POINTER(_ChunkOpts)]),
        "mrt_df_embed_tokens": (i32, [vp, ctypes.POINTER(ctypes.c_int32), i32, vp, vp]),
        "mrt_df_position_embedding": (i32, [vp, i32, vp]),
        "mrt_stream_config_default": (None, [ctypes.POINTER(_StreamConfig)]),
        "mrt_chunk_opts_default": (None, [ctypes.POINTER(_ChunkOpts)]),
        "mrt_df_stream_create": (i32, [vp, ctypes.POINTER(_StreamConfig), ctypes.POINTER(vp)]),
        "mrt_df_stream_destroy": (None, [vp]),
        "mrt_df_stream_generate_chunk": (i32, [vp, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(_ChunkOpts),
                                               ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32)]),
        "mrt_df_stream_set_context": (i32, [vp, ctypes.POINTER(ctypes.c_int32), ctypes.c_int64]),
        "mrt_df_stream_get_context": (i32, [vp, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int64)]),
        "mrt_df_stream_state": (i32, [vp, ctypes.POINTER(vp)]),
        "mrt_df_stream_generate_chunk_audio": (i32, [vp, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(_ChunkOpts),
                                                     ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32),
                                                     ctypes.POINTER(ctypes.c_float)]),
        "mrt_df_stream_attach_codec": (i32, [vp, vp]),
        "mrt_df_batch_create": (i32, [vp, i32, i32, i32, ctypes.POINTER(vp)]),
        "mrt_df_batch_destroy": (None, [vp]),
        "mrt_df_batch_encode": (i32, [vp, ctypes.POINTER(ctypes.c_int32)]),
        "mrt_df_batch_generate_tokens": (i32, [vp, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(_GenOpts),
                                               ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_int32)]),
        "mrt_df_batch_stream": (i32, [vp, ctypes.POINTER(vp)]),
        "mrt_df_batch_decode_time": (i32, [vp, ctypes.POINTER(ctypes.c_float)]),
        "mrt_df_batch_read_enc_out": (i32, [vp, vp, sz]),
        "mrt_codec_config_default": (None, [ctypes.POINTER(_CodecConfig)]),
        "mrt_codec_create": (i32, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(_CodecConfig), i32,
                                   ctypes.POINTER(vp)]),
        "mrt_codec_create_from_tensors": (i32, [i32, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(vp),
                                                ctypes.POINTER(vp), ctypes.POINTER(ctypes.c_int32),
                                                ctypes.POINTER(_CodecConfig), i32, ctypes.POINTER(vp)]),
        "mrt_codec_destroy": (None, [vp]),
        "mrt_codec_decode": (i32, [vp, ctypes.POINTER(ctypes.c_int32), i32, ctypes.POINTER(ctypes.c_float)]),
        "mrt_codec_decode_device": (i32, [vp, vp, i32, vp]),
        "mrt_codec_stream": (i32, [vp, ctypes.POINTER(vp)]),
        "mrt_codec_sync": (i32, [vp]),
        "mrt_codec_decode_time": (i32, [vp, ctypes.POINTER(ctypes.c_float)]),
        "mrt_codec_read": (i32, [vp, i32, vp, sz]),
        "mrt_coca_config_default": (None, [ctypes.POINTER(_CocaConfig)]),
        "mrt_coca_create": (i32, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(_CocaConfig), i32,
                                  ctypes.POINTER(vp)]),
        "mrt_coca_create_from_tensors": (i32, [i32, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(vp),
                                               ctypes.POINTER(vp), ctypes.POINTER(ctypes.c_int32),
                                               ctypes.POINTER(_CocaConfig), i32, ctypes.POINTER(vp)]),
        "mrt_coca_destroy": (None, [vp]),
        "mrt_coca_embed_text": (i32, [vp, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_float),
                                      ctypes.POINTER(ctypes.c_float)]),
        "mrt_coca_tokenize": (i32, [vp, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_int32)]),
        "mrt_coca_style_tokens_lm": (i32, [vp, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_float), i32,
                                           i32, i32, ctypes.POINTER(ctypes.c_int32)]),
        "mrt_coca_embed_time": (i32, [vp, ctypes.POINTER(ctypes.c_float)]),
        "mrt_coca_read": (i32, [vp, i32, vp, sz]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def _check(lib, code: int) -> None:
    if code != MRT_OK:
        raise MrtError(code, lib.mrt_last_error().decode(errors="replace"))


def _i32_ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


def _torch():
    import torch  # noqa: PLC0415  (device allocator only)
    return torch


def _dptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(int(t.data_ptr()))


class Depthformer:
    """Device-resident Depthformer (model.h:72-239)."""

    def __init__(self, weights, config: Config, dtype: str = "bf16", device: int = 0):
        self.lib = load_library()
        self.config = config
        self.dtype = dtype = parse_dtype(dtype)
        self.device = device
        d = _DTYPE_CODE
        h = ctypes.c_void_p()
        cfg = config.to_c()
        if isinstance(weights, (str, os.PathLike)):
            _check(self.lib, self.lib.mrt_df_create(str(weights).encode(), ctypes.byref(cfg), d[dtype],
                                                    device, ctypes.byref(h)))
        else:
            names, arrays = [], []
            for k, v in weights.items():
                names.append(k.encode())
                arrays.append(np.ascontiguousarray(v, dtype=np.float32))
            n = len(names)
            c_names = (ctypes.c_char_p * n)(*names)
            c_data = (ctypes.c_void_p * n)(*[a.ctypes.data for a in arrays])
            shapes = [np.asarray(a.shape, dtype=np.int64) for a in arrays]
            c_shapes = (ctypes.c_void_p * n)(*[s.ctypes.data for s in shapes])
            c_nd = (ctypes.c_int32 * n)(*[a.ndim for a in arrays])
            _check(self.lib, self.lib.mrt_df_create_from_tensors(
                n, c_names, c_data, c_shapes, c_nd, ctypes.byref(cfg), d[dtype], device,
                ctypes.byref(h)))
        self._h = h

    def precompute_biases(self, kind: str, n: int):
        """precompute_{temporal,depth}_biases(n): a list of n device tensors, the
        f-th of shape (H, f + 1) in the model dtype (views of one buffer)."""
        torch = _torch()
        H = self.config.num_heads
        buf = torch.empty(H * n * (n + 1) // 2, dtype=self.torch_dtype, device=f"cuda:{self.device}")
        torch.cuda.synchronize(self.device)
        _check(self.lib, self.lib.mrt_df_precompute_biases(self._h, {"temporal": 0, "depth": 1}[kind], n, _dptr(buf)))
        return [buf[H * f * (f + 1) // 2: H * (f + 1) * (f + 2) // 2].view(H, f + 1) for f in range(n)]

    def token_embedding(self, ids, out=None):
        """Depthformer::token_embedding()(ids) (model.h:127): a (len(ids), d_model)
        device tensor in the model dtype, rows emb[ids] (mrt_df_embed_tokens)."""
        torch = _torch()
        a = np.ascontiguousarray(np.asarray(ids).reshape(-1), dtype=np.int32)
        if out is None:
            out = torch.empty((a.size, self.config.d_model), dtype=self.torch_dtype, device=f"cuda:{self.device}")
        torch.cuda.synchronize(self.device)
        _check(self.lib, self.lib.mrt_df_embed_tokens(self._h, _i32_ptr(a), a.size, _dptr(out), None))
        return out

    def position_embedding(self, seq_len: int):
        """Depthformer::position_embedding(seq_len) (model.cpp:215-224): the fp32
        sinusoid rows (seq_len, d_model) as a device tensor."""
        torch = _torch()
        out = torch.empty((seq_len, self.config.d_model), dtype=torch.float32, device=f"cuda:{self.device}")
        torch.cuda.synchronize(self.device)
        _check(self.lib, self.lib.mrt_df_position_embedding(self._h, seq_len, _dptr(out)))
        return out

    @property
    def torch_dtype(self):
        torch = _torch()
        return {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}[self.dtype]

    def new_state(self, rows: int = 2, max_frames: int = 50, enc_len: Optional[int] = None) -> "State":
        return State(self, rows, max_frames, enc_len or self.config.max_encoder_length)

    def close(self) -> None:
        if getattr(self, "_h", None):
            self.lib.mrt_df_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass


class State:
    """One decode stream: encoder output, cross K/V, ring KV caches, HIP stream."""

    def __init__(self, model: Depthformer, rows: int, max_frames: int, enc_len: int):
        self.model = model
        self.lib = model.lib
        self.rows, self.max_frames, self.enc_len = rows, max_frames, enc_len
        h = ctypes.c_void_p()
        _check(self.lib, self.lib.mrt_df_state_create(model._h, rows, max_frames, enc_len, ctypes.byref(h)))
        self._h = h

    # -- reference methods ------------------------------------------------
    def encode(self, tokens: np.ndarray) -> None:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        if t.shape != (self.rows, self.enc_len):
            raise ValueError(f"tokens must be {(self.rows, self.enc_len)}, got {t.shape}")
        _check(self.lib, self.lib.mrt_df_encode(self._h, _i32_ptr(t)))

    def temporal_step(self, frame_emb, frame_idx: int, enc_out=None, out=None, sync: bool = True,
                      position_bias=None):
        """One temporal step on the state's stream.  With sync=False the call only
        enqueues: the inputs must already be complete and the caller orders later
        reads of `out` after the state's stream.  position_bias: optional (H,
        frame_idx + 1) device tensor in the model dtype (the reference's explicit bias)."""
        torch = _torch()
        if out is None:
            out = torch.empty_like(frame_emb)
        if sync:
            self._sync_torch()
        enc = _dptr(enc_out) if enc_out is not None else None
        if position_bias is None:
            _check(self.lib, self.lib.mrt_df_temporal_step(self._h, _dptr(frame_emb), enc, frame_idx, _dptr(out)))
        else:
            _check(self.lib, self.lib.mrt_df_temporal_step_with_bias(self._h, _dptr(frame_emb), enc, frame_idx,
                                                                     _dptr(position_bias), _dptr(out)))
        if sync:
            self.sync()
        return out

    def depth_step(self, tok_emb, depth_idx: int, level: Optional[int] = None,
                   codebook_size: int = 1024, codec_offset: int = 2, out=None, sync: bool = True,
                   position_bias=None):
        """One depth step; logits of the level slice (or the full vocabulary when
        level is None).  sync=False and position_bias as for temporal_step."""
        torch = _torch()
        cfg = self.model.config
        n = codebook_size if level is not None else cfg.vocab_size
        if out is None:
            out = torch.empty((self.rows, n), dtype=torch.float32, device=tok_emb.device)
        if sync:
            self._sync_torch()
        lv = -1 if level is None else level
        if position_bias is None:
            _check(self.lib, self.lib.mrt_df_depth_step(self._h, _dptr(tok_emb), depth_idx, lv, codebook_size,
                                                        codec_offset, _dptr(out)))
        else:
            _check(self.lib, self.lib.mrt_df_depth_step_with_bias(self._h, _dptr(tok_emb), depth_idx,
                                                                  _dptr(position_bias), lv, codebook_size,
                                                                  codec_offset, _dptr(out)))
        if sync:
            self.sync()
        return out

    def generate_tokens(self, enc_tokens: Optional[np.ndarray], opts: GenOptions,
                        teacher: Optional[np.ndarray] = None, record: Optional[Dict] = None) -> np.ndarray:
        o = self._opts(opts)
        keep = []
        if teacher is not None:
            tt = np.ascontiguousarray(teacher, dtype=np.int32)
            if tt.shape != (opts.num_frames, opts.rvq_depth):
                raise ValueError("teacher must be (num_frames, rvq_depth)")
            keep.append(tt)
            o.teacher = _i32_ptr(tt)
        if record is not None:
            for key, field in (("slices", "record_slices"), ("temporal", "record_temporal"),
                               ("drawn", "record_drawn"), ("frame_mean", "record_frame_mean")):
                if key in record:
                    setattr(o, field, int(record[key].data_ptr()))
            self._sync_torch()
        enc = None
        if enc_tokens is not None:
            enc = np.ascontiguousarray(enc_tokens, dtype=np.int32)
            if enc.shape != (self.rows, self.enc_len):
                raise ValueError(f"enc_tokens must be {(self.rows, self.enc_len)}")
        out = np.zeros((opts.num_frames, opts.rvq_depth), dtype=np.int32)
        _check(self.lib, self.lib.mrt_df_generate_tokens(
            self._h, _i32_ptr(enc) if enc is not None else None, ctypes.byref(o), _i32_ptr(out)))
        return out

    def sample_level(self, slice_logits, opts: GenOptions, frame: int, level: int) -> int:
        o = self._opts(opts)
        tok = ctypes.c_int32()
        self._sync_torch()
        _check(self.lib, self.lib.mrt_df_sample_level(self._h, _dptr(slice_logits), ctypes.byref(o),
                                                      frame, level, ctypes.byref(tok)))
        return int(tok.value)

    # -- buffers ------------------------------------------------------------
    def buffer_shape(self, which: int):
        c = self.model.config
        H = c.num_heads
        return {
            BUF_ENC_OUT: (self.rows, self.enc_len, c.d_model),
            BUF_CROSS_K: (self.rows, H, self.enc_len, 64), BUF_CROSS_V: (self.rows, H, self.enc_len, 64),
            BUF_TEMPORAL_K: (self.rows, H, self.max_frames, 64),
            BUF_TEMPORAL_V: (self.rows, H, self.max_frames, 64),
            BUF_DEPTH_K: (self.rows, H, c.rvq_depth, 64), BUF_DEPTH_V: (self.rows, H, c.rvq_depth, 64),
            BUF_ENC_TOKENS: (self.rows, self.enc_len),
        }[which]

    def read(self, which: int, layer: int = 0):
        torch = _torch()
        dt = torch.int32 if which == BUF_ENC_TOKENS else self.model.torch_dtype
        t = torch.empty(self.buffer_shape(which), dtype=dt, device=f"cuda:{self.model.device}")
        self._sync_torch()
        _check(self.lib, self.lib.mrt_df_state_read(self._h, which, layer, _dptr(t),
                                                    t.numel() * t.element_size()))
        return t

    def write(self, which: int, layer: int, t) -> None:
        self._sync_torch()
        _check(self.lib, self.lib.mrt_df_state_write(self._h, which, layer, _dptr(t),
                                                     t.numel() * t.element_size()))

    def set_cache_length(self, kind: int, length: int) -> None:
        _check(self.lib, self.lib.mrt_df_state_set_cache_length(self._h, kind, length))

    def reset_cache(self, kind: str) -> None:
        """Empty the "temporal" or "depth" KV cache (empty_*_cache)."""
        _check(self.lib, self.lib.mrt_df_state_reset_cache(self._h, {"temporal": 0, "depth": 1}[kind]))

    def depth_forward_full(self, embs, position_bias=None, causal: bool = True):
        """Depthformer::depth_forward_full: embs (2, k, d_model) device tensor in
        the model dtype -> (2, k, vocab) fp32 logits (a new device tensor).
        position_bias: None (the k x k rel-pos block) or (H, k, k) device tensor."""
        torch = _torch()
        k = int(embs.shape[1])
        out = torch.empty((2, k, self.model.config.vocab_size), dtype=torch.float32,
                          device=f"cuda:{self.model.device}")
        self._sync_torch()
        _check(self.lib, self.lib.mrt_df_depth_forward_full(
            self._h, _dptr(embs.contiguous()), k, _dptr(position_bias.contiguous()) if position_bias is not None else None,
            1 if causal else 0, _dptr(out)))
        return out

    def decode_time(self):
        """(GPU ms, persistent launches) of the decode section of the last
        generate_tokens call, timed with HIP events on the state's stream."""
        ms, n = ctypes.c_float(), ctypes.c_int()
        _check(self.lib, self.lib.mrt_df_state_decode_time(self._h, ctypes.byref(ms), ctypes.byref(n)))
        return float(ms.value), int(n.value)

    def phase_trace(self):
        """(raw stamps (2, 512) uint64, clock MHz) of the last decode's frame 1
        (temporal step, depth level 1), recorded when MRT_TRACE_PHASES was set
        at state creation (mrt_df_state_phase_trace)."""
        buf = (ctypes.c_uint64 * 1024)()
        mhz = ctypes.c_float()
        _check(self.lib, self.lib.mrt_df_state_phase_trace(self._h, buf, 1024, ctypes.byref(mhz)))
        return np.frombuffer(buf, dtype=np.uint64).reshape(2, 512).copy(), float(mhz.value)

    def compile_for_inference(self, opts: GenOptions) -> None:
        """Depthformer::compile_for_inference for this state's decode with
        ``opts`` (mrt_df_state_compile): the q/k/v table, the captured graph and
        the first launch of every kernel happen here, not in the first chunk."""
        o = self._opts(opts)
        _check(self.lib, self.lib.mrt_df_state_compile(self._h, ctypes.byref(o)))

    def set_profile(self, on: bool = True) -> None:
        """Phase stamps of the frame kernel for later decodes (mrt_df_state_set_profile)."""
        _check(self.lib, self.lib.mrt_df_state_set_profile(self._h, 1 if on else 0))

    def decode_profile(self) -> dict:
        """The MRT_PROFILE_DECODE split of the last generate_tokens call (GPU ms):
        total, encoder, bias, temporal, depth, sample; -1 where not recorded."""
        p = _DecodeProfile()
        _check(self.lib, self.lib.mrt_df_state_decode_profile(self._h, ctypes.byref(p)))
        return {n: (int(getattr(p, n)) if n == "frames" else float(getattr(p, n))) for n, _ in p._fields_}

    def spec_acceptance(self) -> float:
        """Share of the last generate_tokens call's levels taken from the
        speculative verification pass (-1: it did not speculate)."""
        a = ctypes.c_float()
        _check(self.lib, self.lib.mrt_df_state_spec_acceptance(self._h, ctypes.byref(a)))
        return float(a.value)

    def stream_handle(self) -> int:
        s = ctypes.c_void_p()
        _check(self.lib, self.lib.mrt_df_state_stream(self._h, ctypes.byref(s)))
        return int(s.value or 0)

    def sync(self) -> None:
        _check(self.lib, self.lib.mrt_df_sync(self._h))

    def close(self) -> None:
        if getattr(self, "_h", None):
            if not getattr(self, "_borrowed", False):
                self.lib.mrt_df_state_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass

    @classmethod
    def _view(cls, model: Depthformer, handle: ctypes.c_void_p, rows: int, max_frames: int,
              enc_len: int) -> "State":
        """A handle owned elsewhere (a stream's state); close() leaves it alone."""
        st = cls.__new__(cls)
        st.model, st.lib = model, model.lib
        st.rows, st.max_frames, st.enc_len = rows, max_frames, enc_len
        st._h, st._borrowed = handle, True
        return st

    # -- helpers --------------------------------------------------------------
    @staticmethod
    def _opts(opts: GenOptions) -> _GenOpts:
        return _GenOpts(num_frames=opts.num_frames, rvq_depth=opts.rvq_depth,
                        temperature=opts.temperature, top_k=opts.top_k,
                        guidance_weight=opts.guidance_weight, seed=opts.seed & ((1 << 64) - 1),
                        codebook_size=opts.codebook_size, codec_offset=opts.codec_offset,
                        teacher=None, use_graph=1 if opts.use_graph else 0,
                        speculative=1 if getattr(opts, "speculative", False) else 0)

    @staticmethod
    def _sync_torch() -> None:
        torch = _torch()
        if torch.cuda.is_available():
            torch.cuda.synchronize()


@dataclasses.dataclass(frozen=True)
class StreamConfig:
    """The SystemConfig fields of the token half (system.h:44-83)."""

    chunk_frames: int = 50
    context_frames: int = 250
    codebook_size: int = 1024
    encoder_codec_rvq_depth: int = 4
    encoder_style_rvq_depth: int = 6
    decoder_codec_rvq_depth: int = 16
    mask_token: int = 1
    codec_offset: int = 2
    crossfade_frames: int = 1
    samples_per_frame: int = 1920

    @property
    def encoder_length(self) -> int:
        return self.context_frames * self.encoder_codec_rvq_depth + self.encoder_style_rvq_depth

    def to_c(self) -> _StreamConfig:
        return _StreamConfig(*[getattr(self, f) for f, _ in _StreamConfig._fields_])


@dataclasses.dataclass
class ChunkOptions:
    """GenerateChunkOptions (system.h:86-121)."""

    temperature: float = 1.1
    top_k: int = 40
    guidance_weight: float = 5.0
    seed: Optional[int] = None
    pipeline_encoder: bool = False
    use_graph: bool = True
    speculative: int = 0  # 0 off, 1 on, 2 adaptive (see mrt_chunk_opts)


class Stream:
    """System::generate_chunk's token half with the RVQ context on the device
    (system.cpp:177-370): encoder inputs, encoder, decode, llm_to_rvq and the
    context roll all run on the stream's HIP stream."""

    def __init__(self, model: Depthformer, cfg: StreamConfig = StreamConfig()):
        self.model, self.lib, self.cfg = model, model.lib, cfg
        h = ctypes.c_void_p()
        c = cfg.to_c()
        _check(self.lib, self.lib.mrt_df_stream_create(model._h, ctypes.byref(c), ctypes.byref(h)))
        self._h = h
        sh = ctypes.c_void_p()
        _check(self.lib, self.lib.mrt_df_stream_state(h, ctypes.byref(sh)))
        self.state = State._view(model, sh, 2, cfg.chunk_frames, cfg.encoder_length)

    def attach_codec(self, codec: Optional["Codec"]) -> None:
        """Decode each chunk's codes to audio with ``codec`` (None detaches)."""
        _check(self.lib, self.lib.mrt_df_stream_attach_codec(self._h, codec._h if codec is not None else None))
        self._codec = codec  # kept alive while attached

    def generate_chunk_audio(self, style: Optional[Sequence[int]], opts: ChunkOptions,
                             teacher: Optional[np.ndarray] = None):
        """The whole System::generate_chunk: (llm ids, rvq codes, audio
        (chunk_frames * samples_per_frame, 2) float32)."""
        return self.generate_chunk(style, opts, teacher, audio=True)

    @staticmethod
    def _chunk_opts(opts: ChunkOptions) -> _ChunkOpts:
        return _ChunkOpts(temperature=opts.temperature, top_k=opts.top_k, guidance_weight=opts.guidance_weight,
                          has_seed=0 if opts.seed is None else 1,
                          seed=0 if opts.seed is None else opts.seed & ((1 << 64) - 1),
                          pipeline_encoder=1 if opts.pipeline_encoder else 0,
                          use_graph=1 if opts.use_graph else 0, teacher=None,
                          speculative=int(opts.speculative))

    def compile_for_inference(self, opts: ChunkOptions) -> None:
        """compile_for_inference for this stream's chunks (mrt_df_stream_compile,
        system.cpp:130): the first chunk then pays no one-time work."""
        o = self._chunk_opts(opts)
        _check(self.lib, self.lib.mrt_df_stream_compile(self._h, ctypes.byref(o)))

    def generate_chunk(self, style: Optional[Sequence[int]], opts: ChunkOptions,
                       teacher: Optional[np.ndarray] = None, audio: bool = False):
        """Returns (llm ids, rvq codes), both (chunk_frames, levels) int32
        (and the chunk's audio with ``audio``)."""
        cfg = self.cfg
        shape = (cfg.chunk_frames, cfg.decoder_codec_rvq_depth)
        o = self._chunk_opts(opts)
        keep = []
        if teacher is not None:
            tt = np.ascontiguousarray(teacher, dtype=np.int32)
            if tt.shape != shape:
                raise ValueError(f"teacher must be {shape}")
            keep.append(tt)
            o.teacher = _i32_ptr(tt)
        st = None
        if style is not None:
            st = np.ascontiguousarray(style, dtype=np.int32)
            if st.shape != (cfg.encoder_style_rvq_depth,):
                raise ValueError("style_tokens_lm size != encoder_style_rvq_depth")
        llm = np.zeros(shape, dtype=np.int32)
        rvq = np.zeros(shape, dtype=np.int32)
        if audio:
            wav = np.zeros((cfg.chunk_frames * cfg.samples_per_frame, 2), dtype=np.float32)
            _check(self.lib, self.lib.mrt_df_stream_generate_chunk_audio(
                self._h, _i32_ptr(st) if st is not None else None, ctypes.byref(o), _i32_ptr(llm), _i32_ptr(rvq),
                wav.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
            return llm, rvq, wav
        _check(self.lib, self.lib.mrt_df_stream_generate_chunk(
            self._h, _i32_ptr(st) if st is not None else None, ctypes.byref(o), _i32_ptr(llm), _i32_ptr(rvq)))
        return llm, rvq

    def set_context(self, context: np.ndarray, chunk_index: int = 0) -> None:
        c = np.ascontiguousarray(context, dtype=np.int32)
        if c.shape != (self.cfg.context_frames, self.cfg.decoder_codec_rvq_depth):
            raise ValueError("context must be (context_frames, decoder_codec_rvq_depth)")
        _check(self.lib, self.lib.mrt_df_stream_set_context(self._h, _i32_ptr(c), chunk_index))

    def get_context(self):
        """(context (context_frames, levels) int32, chunk index)."""
        c = np.zeros((self.cfg.context_frames, self.cfg.decoder_codec_rvq_depth), dtype=np.int32)
        idx = ctypes.c_int64()
        _check(self.lib, self.lib.mrt_df_stream_get_context(self._h, _i32_ptr(c), ctypes.byref(idx)))
        return c, int(idx.value)

    @property
    def chunk_index(self) -> int:
        idx = ctypes.c_int64()
        _check(self.lib, self.lib.mrt_df_stream_get_context(self._h, None, ctypes.byref(idx)))
        return int(idx.value)

    def close(self) -> None:
        if getattr(self, "_h", None):
            self.state._h = None
            self.lib.mrt_df_stream_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass


class Batch:
    """Independent streams decoded together (2 rows per stream, <= 32 streams,
    bf16): per stream the semantics of State.generate_tokens."""

    def __init__(self, model: Depthformer, streams: int, max_frames: int = 50, enc_len: Optional[int] = None):
        self.model, self.lib = model, model.lib
        self.streams, self.max_frames = streams, max_frames
        self.enc_len = enc_len or model.config.max_encoder_length
        h = ctypes.c_void_p()
        _check(self.lib, self.lib.mrt_df_batch_create(model._h, streams, max_frames, self.enc_len, ctypes.byref(h)))
        self._h = h

    def encode(self, tokens: np.ndarray) -> None:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        if t.shape != (2 * self.streams, self.enc_len):
            raise ValueError(f"tokens must be {(2 * self.streams, self.enc_len)}")
        _check(self.lib, self.lib.mrt_df_batch_encode(self._h, _i32_ptr(t)))

    def generate_tokens(self, enc_tokens: Optional[np.ndarray], opts: GenOptions, seeds: Sequence[int],
                        teacher: Optional[np.ndarray] = None, record: Optional[Dict] = None) -> np.ndarray:
        """(streams, num_frames, rvq_depth) LLM ids; stream s draws with seeds[s]."""
        o = State._opts(opts)
        keep = []
        sd = np.ascontiguousarray([int(x) & ((1 << 64) - 1) for x in seeds], dtype=np.uint64)
        if sd.shape != (self.streams,):
            raise ValueError("one seed per stream")
        if teacher is not None:
            tt = np.ascontiguousarray(teacher, dtype=np.int32)
            if tt.shape != (self.streams, opts.num_frames, opts.rvq_depth):
                raise ValueError("teacher must be (streams, num_frames, rvq_depth)")
            keep.append(tt)
            o.teacher = _i32_ptr(tt)
        if record is not None:
            for key, field in (("slices", "record_slices"), ("temporal", "record_temporal")):
                if key in record:
                    setattr(o, field, int(record[key].data_ptr()))
            State._sync_torch()
        enc = None
        if enc_tokens is not None:
            enc = np.ascontiguousarray(enc_tokens, dtype=np.int32)
            if enc.shape != (2 * self.streams, self.enc_len):
                raise ValueError(f"enc_tokens must be {(2 * self.streams, self.enc_len)}")
        out = np.zeros((self.streams, opts.num_frames, opts.rvq_depth), dtype=np.int32)
        _check(self.lib, self.lib.mrt_df_batch_generate_tokens(
            self._h, _i32_ptr(enc) if enc is not None else None, ctypes.byref(o),
            sd.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)), _i32_ptr(out)))
        return out

    def decode_time(self) -> float:
        ms = ctypes.c_float()
        _check(self.lib, self.lib.mrt_df_batch_decode_time(self._h, ctypes.byref(ms)))
        return float(ms.value)

    def stream_handle(self) -> int:
        s = ctypes.c_void_p()
        _check(self.lib, self.lib.mrt_df_batch_stream(self._h, ctypes.byref(s)))
        return int(s.value or 0)

    def read_enc_out(self):
        torch = _torch()
        t = torch.empty((2 * self.streams, self.enc_len, self.model.config.d_model), dtype=torch.bfloat16,
                        device=f"cuda:{self.model.device}")
        State._sync_torch()
        _check(self.lib, self.lib.mrt_df_batch_read_enc_out(self._h, _dptr(t), t.numel() * 2))
        return t

    def close(self) -> None:
        if getattr(self, "_h", None):
            self.lib.mrt_df_batch_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass


def _tensor_list(weights):
    names, arrays = [], []
    for k, v in weights.items():
        names.append(k.encode())
        arrays.append(np.ascontiguousarray(v, dtype=np.float32))
    n = len(names)
    shapes = [np.asarray(a.shape, dtype=np.int64) for a in arrays]
    keep = (arrays, shapes)
    return (n, (ctypes.c_char_p * n)(*names), (ctypes.c_void_p * n)(*[a.ctypes.data for a in arrays]),
            (ctypes.c_void_p * n)(*[x.ctypes.data for x in shapes]), (ctypes.c_int32 * n)(*[a.ndim for a in arrays]),
            keep)


class Codec:
    """Codec decode on the device (system.cpp:373-390): RVQ ids (frames, 16)
    -> rvq_dequantization -> SpectroStreamDecoder -> istft_postprocess ->
    stereo audio (frames * 1920, 2) float32 at 48 kHz.

    ``weights``: a dict holding the decoder keys and "codebooks", or a pair of
    paths (spectrostream_decoder.safetensors, spectrostream_codebooks.safetensors).
    ``channels``: optional (embedding_dim, proj_channels, block_in, block_out)
    for a reduced test decoder; the default is the reference's."""

    def __init__(self, weights, max_frames: int = 51, device: int = 0, channels=None, rvq_levels: int = 16,
                 codebook_size: int = 1024):
        self.lib = load_library()
        cfg = _CodecConfig()
        self.lib.mrt_codec_config_default(ctypes.byref(cfg))
        if channels is not None:
            e, p, bi, bo = channels
            cfg.embedding_dim, cfg.proj_channels = e, p
            for i in range(7):
                cfg.block_in[i], cfg.block_out[i] = bi[i], bo[i]
        cfg.rvq_levels, cfg.codebook_size, cfg.max_frames = rvq_levels, codebook_size, max_frames
        self.max_frames, self.levels = max_frames, rvq_levels
        h = ctypes.c_void_p()
        if isinstance(weights, (tuple, list)):
            _check(self.lib, self.lib.mrt_codec_create(str(weights[0]).encode(), str(weights[1]).encode(),
                                                       ctypes.byref(cfg), device, ctypes.byref(h)))
        else:
            n, c_names, c_data, c_shapes, c_nd, _keep = _tensor_list(weights)
            _check(self.lib, self.lib.mrt_codec_create_from_tensors(n, c_names, c_data, c_shapes, c_nd,
                                                                    ctypes.byref(cfg), device, ctypes.byref(h)))
        self._h = h

    def decode(self, rvq_tokens: np.ndarray) -> np.ndarray:
        tok = np.ascontiguousarray(rvq_tokens, dtype=np.int32)
        if tok.ndim != 2 or tok.shape[1] != self.levels:
            raise ValueError(f"rvq_tokens must be (frames, {self.levels})")
        out = np.empty((tok.shape[0] * 1920, 2), dtype=np.float32)
        _check(self.lib, self.lib.mrt_codec_decode(self._h, _i32_ptr(tok), tok.shape[0],
                                                   out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
        return out

    def decode_device(self, tokens_dev, audio_dev) -> None:
        """Device tensors: tokens (frames, levels) int32, audio (frames * 1920, 2) float32."""
        _check(self.lib, self.lib.mrt_codec_decode_device(self._h, _dptr(tokens_dev), int(tokens_dev.shape[0]),
                                                          _dptr(audio_dev)))

    def sync(self) -> None:
        _check(self.lib, self.lib.mrt_codec_sync(self._h))

    def stream_handle(self) -> int:
        s = ctypes.c_void_p()
        _check(self.lib, self.lib.mrt_codec_stream(self._h, ctypes.byref(s)))
        return int(s.value or 0)

    def decode_time(self) -> float:
        ms = ctypes.c_float()
        _check(self.lib, self.lib.mrt_codec_decode_time(self._h, ctypes.byref(ms)))
        return float(ms.value)

    def read(self, which: int, shape) -> np.ndarray:
        out = np.empty(shape, dtype=np.float32)
        _check(self.lib, self.lib.mrt_codec_read(self._h, which, ctypes.c_void_p(out.ctypes.data), out.nbytes))
        return out

    def close(self) -> None:
        if getattr(self, "_h", None):
            self.lib.mrt_codec_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass


@dataclasses.dataclass(frozen=True)
class CocaConfig:
    """MusicCoCaConfig (musiccoca.h:151-162) + the StyleModel constants."""

    d_model: int = 768
    num_heads: int = 12
    d_head: int = 64
    d_ff: int = 3072
    num_layers: int = 12
    pooler_d_head: int = 256
    vocab_size: int = 64000
    max_text_len: int = 128
    rvq_depth: int = 12
    codebook_size: int = 1024

    @staticmethod
    def tiny() -> "CocaConfig":
        return CocaConfig(d_model=128, num_heads=4, d_head=32, d_ff=256, num_layers=2, pooler_d_head=64,
                          vocab_size=500, max_text_len=32, rvq_depth=12, codebook_size=64)

    def to_c(self) -> _CocaConfig:
        return _CocaConfig(*[getattr(self, f) for f, _ in _CocaConfig._fields_])


class StyleModel:
    """StyleModel (style_model.h:22-79) on the device: text prompt -> MusicCoCa
    embedding -> RVQ tokens -> LLM-vocabulary style ids.  ``weights``: a dict
    with the text-path keys and "codebooks", or (encoder_path,
    codebooks_path).  ``vocab_path``: a SentencePiece model for string
    prompts (``style_tokens_lm(prompt)``); id arrays work without one."""

    def __init__(self, weights, cfg: CocaConfig = CocaConfig(), device: int = 0, vocab_path=None):
        self.lib, self.cfg = load_library(), cfg
        c = cfg.to_c()
        h = ctypes.c_void_p()
        if isinstance(weights, (tuple, list)):
            _check(self.lib, self.lib.mrt_coca_create(str(weights[0]).encode(), str(weights[1]).encode(),
                                                      ctypes.byref(c), device, ctypes.byref(h)))
        else:
            n, c_names, c_data, c_shapes, c_nd, _keep = _tensor_list(weights)
            _check(self.lib, self.lib.mrt_coca_create_from_tensors(n, c_names, c_data, c_shapes, c_nd,
                                                                   ctypes.byref(c), device, ctypes.byref(h)))
        self._h = h
        self._spm = None
        if vocab_path is not None:
            import sentencepiece  # noqa: PLC0415  (host tokenizer, as the reference links it)
            self._spm = sentencepiece.SentencePieceProcessor(model_file=str(vocab_path))

    def text_ids(self, prompt: str):
        """StyleModel::tokenize_text_ids (style_model.cpp:52-74)."""
        if self._spm is None:
            raise RuntimeError("no SentencePiece vocabulary: pass vocab_path or use ids")
        raw = self._spm.encode(prompt.lower())
        L = self.cfg.max_text_len
        keep = min(len(raw), L - 1)
        ids = np.zeros(L, np.int32)
        pad = np.ones(L, np.float32)
        ids[0], pad[0] = 1, 0
        ids[1:keep + 1], pad[1:keep + 1] = raw[:keep], 0
        return ids, pad

    def embed_text(self, ids: np.ndarray, padding: np.ndarray) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        pad = np.ascontiguousarray(padding, dtype=np.float32)
        if ids.shape != (self.cfg.max_text_len,) or pad.shape != ids.shape:
            raise ValueError(f"ids / padding must be ({self.cfg.max_text_len},)")
        out = np.empty(self.cfg.d_model, np.float32)
        _check(self.lib, self.lib.mrt_coca_embed_text(self._h, _i32_ptr(ids),
                                                      pad.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                                      out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
        return out

    def tokenize(self, embedding: Optional[np.ndarray] = None) -> np.ndarray:
        tok = np.empty(self.cfg.rvq_depth, np.int32)
        e = None
        if embedding is not None:
            e = np.ascontiguousarray(embedding, dtype=np.float32)
            if e.shape != (self.cfg.d_model,):
                raise ValueError(f"embedding must be ({self.cfg.d_model},)")
        _check(self.lib, self.lib.mrt_coca_tokenize(
            self._h, e.ctypes.data_as(ctypes.POINTER(ctypes.c_float)) if e is not None else None, _i32_ptr(tok)))
        return tok

    def style_tokens_lm(self, prompt, style_depth: int = 6, codebook: int = 1024, offset: int = 17410,
                        padding: Optional[np.ndarray] = None) -> np.ndarray:
        """``prompt``: a string (needs the vocabulary) or an ids array with ``padding``."""
        if isinstance(prompt, str):
            ids, padding = self.text_ids(prompt)
        else:
            ids = prompt
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        pad = np.ascontiguousarray(padding, dtype=np.float32)
        out = np.empty(style_depth, np.int32)
        _check(self.lib, self.lib.mrt_coca_style_tokens_lm(self._h, _i32_ptr(ids),
                                                           pad.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                                           style_depth, codebook, offset, _i32_ptr(out)))
        return out

    def embed_time(self) -> float:
        ms = ctypes.c_float()
        _check(self.lib, self.lib.mrt_coca_embed_time(self._h, ctypes.byref(ms)))
        return float(ms.value)

    def read(self, which: int, shape) -> np.ndarray:
        out = np.empty(shape, dtype=np.float32)
        _check(self.lib, self.lib.mrt_coca_read(self._h, which, ctypes.c_void_p(out.ctypes.data), out.nbytes))
        return out

    def close(self) -> None:
        if getattr(self, "_h", None):
            self.lib.mrt_coca_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001
            pass
