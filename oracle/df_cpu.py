"""ctypes wrapper of df_cpu.c, the C/OpenMP restatement of one chunk's
streaming decode (encoder, cross K/V, temporal / depth steps, the sampling
loop) in float32 or bf16-emulating precision.

TEST INFRASTRUCTURE ONLY: checked against the numpy oracle in
tests/test_oracle_c.py, used as the fast checker of the chunk-level parity
tests, and timed as the CPU baseline by bench.py.  ``build()`` compiles
``oracle/libdf_cpu.so`` with gcc (OpenMP, AVX2/FMA code generation, no
contraction of separate multiplies and adds).
"""

from __future__ import annotations

import ctypes
import pathlib
import subprocess
from typing import Dict, Optional

import numpy as np

from . import depthformer_oracle as O

HERE = pathlib.Path(__file__).resolve().parent
SRC = HERE / "df_cpu.c"
LIB = HERE / "libdf_cpu.so"


def build() -> pathlib.Path:
    cmd = ["gcc", "-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fopenmp", "-shared", "-fPIC", "-Wall",
           str(SRC), "-o", str(LIB) + ".tmp", "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"df_cpu build failed:\n{' '.join(cmd)}\n{r.stderr}")
    pathlib.Path(str(LIB) + ".tmp").replace(LIB)
    return LIB


class _Stack(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("L", "D", "HD", "H", "F", "cross")] + \
               [(n, ctypes.c_void_p) for n in ("norm_sa", "wq", "wk", "wv", "wo", "norm_ca", "cq", "co",
                                               "norm_ff", "wi0", "wi1", "wo2", "bias_tab", "buckets")]


class _Encoder(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("L", "D", "HD", "H", "F", "V", "max_len")] + \
               [(n, ctypes.c_void_p) for n in ("norm_attn", "wq", "wk", "wv", "wo", "norm_ff", "wi0", "wi1", "wo2",
                                               "enc_norm", "emb", "pe")]


_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists() or LIB.stat().st_mtime < SRC.stat().st_mtime:
            build()
        lib = ctypes.CDLL(str(LIB))
        p, i, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        lib.df_set_threads.argtypes = [i]
        lib.df_set_mode.argtypes = [i]
        lib.df_max_threads.restype = i
        lib.df_temporal_step.argtypes = [ctypes.POINTER(_Stack), p, i, p, p, i, p, p, i, p]
        lib.df_depth_step.argtypes = [ctypes.POINTER(_Stack), p, i, p, p, i, p, p, i, p]
        lib.df_round_bf16.argtypes = [p, ctypes.c_size_t]
        lib.df_encode.argtypes = [ctypes.POINTER(_Encoder), p, i, i, p]
        lib.df_cross_kv.argtypes = [p, i, i, i, i, p, p, p, p]
        lib.df_generate.argtypes = [ctypes.POINTER(_Stack), ctypes.POINTER(_Stack), p, p, p, i, i, i, i, f, f, i,
                                    ctypes.c_uint64, p, p, p, i, p, p, p, p, i, p, p, p, p, p]
        _lib = lib
    return _lib


def _ptr(a: Optional[np.ndarray]) -> Optional[int]:
    return None if a is None else a.ctypes.data


class CpuDepthformer:
    """One CFG pair's decode of a Depthformer bundle (the oracle's weight dict)
    in ``mode`` "fp32" or "bf16" (weights rounded to bf16, every op output
    rounded as the numpy oracle's bf16 mode rounds it)."""

    def __init__(self, weights: Dict[str, np.ndarray], cfg: O.DepthformerConfig, max_frames: int = 50,
                 mode: str = "fp32"):
        if mode not in ("fp32", "bf16"):
            raise ValueError(f"unknown mode {mode!r}")
        self.lib = load()
        self.cfg = cfg
        self.mode = mode
        def f32(k):
            a = np.array(weights[k], dtype=np.float32, order="C", copy=True)
            if mode == "bf16":
                self.lib.df_round_bf16(_ptr(a), a.size)
            return a
        self.keep = []

        def stacked(family, n, key):
            a = np.ascontiguousarray(np.stack([f32(f"{family}.{i}.{key}.weight") for i in range(n)]))
            self.keep.append(a)
            return a

        def stack(family, n, cross):
            st = lambda key: _ptr(stacked(family, n, key))
            table = f32(("temporal" if cross else "depth") + "_rel_pos.relative_attention_bias.weight")
            nb = cfg.temporal_num_buckets if cross else cfg.depth_num_buckets
            md = cfg.temporal_max_distance if cross else cfg.depth_max_distance
            # bucket of query-key distance n (unidirectional: relative position -n)
            bk = np.ascontiguousarray(
                O.relative_position_bucket(-np.arange(4096), False, nb, md).astype(np.int32))
            self.keep += [table, bk]
            s = _Stack(n, cfg.d_model, cfg.num_heads * cfg.d_kv, cfg.num_heads, cfg.d_ff, 1 if cross else 0,
                       st("pre_self_attn_norm"), st("self_attn.q_proj"), st("self_attn.k_proj"),
                       st("self_attn.v_proj"), st("self_attn.o_proj"),
                       st("pre_cross_attn_norm") if cross else None, st("cross_attn.q_proj") if cross else None,
                       st("cross_attn.o_proj") if cross else None, st("pre_ffn_norm"), st("ffn.wi_0"),
                       st("ffn.wi_1"), st("ffn.wo"), _ptr(table), _ptr(bk))
            return s

        self.tstack = stack("temporal_layers", cfg.num_temporal_layers, True)
        self.dstack = stack("depth_layers", cfg.num_depth_layers, False)
        self.dec_norm = f32("decoder_norm.weight")
        self.lm_head = f32("lm_head.weight")
        self.emb = f32("token_embedding.weight")
        self.ckw = stacked("temporal_layers", cfg.num_temporal_layers, "cross_attn.k_proj")
        self.cvw = stacked("temporal_layers", cfg.num_temporal_layers, "cross_attn.v_proj")
        self._weights, self._f32 = weights, f32
        self._enc: Optional[_Encoder] = None
        self.F = max_frames
        H = cfg.num_heads
        self.tk = np.zeros((cfg.num_temporal_layers, 2, H, max_frames, 64), np.float32)
        self.tv = np.zeros_like(self.tk)
        self.dk = np.zeros((cfg.num_depth_layers, 2, H, cfg.rvq_depth, 64), np.float32)
        self.dv = np.zeros_like(self.dk)
        self.ck: Optional[np.ndarray] = None
        self.cv: Optional[np.ndarray] = None

    def _mode(self) -> None:
        self.lib.df_set_mode(1 if self.mode == "bf16" else 0)

    @staticmethod
    def set_threads(n: int) -> None:
        load().df_set_threads(int(n))

    def _encoder(self) -> _Encoder:
        if self._enc is None:
            c = self.cfg
            st = lambda key: _ptr(self._stack_enc(key))
            self.pe = np.ascontiguousarray(O.sinusoidal_position_embedding(c.max_encoder_length, c.d_model))
            self.enc_norm = self._f32("encoder_norm.weight")
            self._enc = _Encoder(c.num_encoder_layers, c.d_model, c.num_heads * c.d_kv, c.num_heads, c.d_ff,
                                 c.vocab_size, c.max_encoder_length,
                                 st("pre_attn_norm"), st("self_attn.q_proj"), st("self_attn.k_proj"),
                                 st("self_attn.v_proj"), st("self_attn.o_proj"), st("pre_ffn_norm"),
                                 st("ffn.wi_0"), st("ffn.wi_1"), st("ffn.wo"), _ptr(self.enc_norm),
                                 _ptr(self.emb), _ptr(self.pe))
        return self._enc

    def _stack_enc(self, key):
        a = np.ascontiguousarray(np.stack([self._f32(f"encoder_layers.{i}.{key}.weight")
                                           for i in range(self.cfg.num_encoder_layers)]))
        self.keep.append(a)
        return a

    def encode(self, tokens: np.ndarray) -> np.ndarray:
        """Depthformer::encode of (2, S) ids -> (2, S, D)."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        assert t.ndim == 2 and t.shape[1] <= self.cfg.max_encoder_length
        assert t.min() >= 0 and t.max() < self.cfg.vocab_size
        out = np.empty((t.shape[0], t.shape[1], self.cfg.d_model), np.float32)
        self._mode()
        self.lib.df_encode(ctypes.byref(self._encoder()), _ptr(t), t.shape[0], t.shape[1], _ptr(out))
        return out

    def set_cross_from_encoder(self, enc: np.ndarray) -> None:
        """precompute_cross_kv of every temporal layer from a (2, S, D) encoder output."""
        e = np.ascontiguousarray(enc, dtype=np.float32)
        c = self.cfg
        S, HD = e.shape[1], c.num_heads * c.d_kv
        self.ck = np.empty((c.num_temporal_layers, 2, c.num_heads, S, 64), np.float32)
        self.cv = np.empty_like(self.ck)
        self._mode()
        self.lib.df_cross_kv(_ptr(e), S, c.num_temporal_layers, c.d_model, HD, _ptr(self.ckw), _ptr(self.cvw),
                             _ptr(self.ck), _ptr(self.cv))

    def set_cross(self, cross_kv) -> None:
        """cross K/V of every temporal layer: the oracle's precompute_cross_kv
        output, a list of (k, v) of shape (2, H, S, 64)."""
        self.ck = np.ascontiguousarray(np.stack([k for k, _ in cross_kv]), dtype=np.float32)
        self.cv = np.ascontiguousarray(np.stack([v for _, v in cross_kv]), dtype=np.float32)

    def temporal_step(self, x: np.ndarray, frame_idx: int) -> np.ndarray:
        assert self.ck is not None and 0 <= frame_idx < self.F
        xin = np.ascontiguousarray(x, dtype=np.float32).reshape(2, self.cfg.d_model)
        out = np.empty_like(xin)
        self._mode()
        self.lib.df_temporal_step(ctypes.byref(self.tstack), _ptr(xin), frame_idx, _ptr(self.tk), _ptr(self.tv),
                                  self.F, _ptr(self.ck), _ptr(self.cv), self.ck.shape[3], _ptr(out))
        return out

    def depth_step(self, x: np.ndarray, depth_idx: int, level: Optional[int] = None, codebook: int = 1024,
                   codec_offset: int = 2) -> np.ndarray:
        D = self.cfg.d_model
        xin = np.ascontiguousarray(x, dtype=np.float32).reshape(2, D)
        if level is None:
            head, rows = self.lm_head, self.cfg.vocab_size
        else:
            head, rows = self.lm_head[codec_offset + codebook * level:], codebook
        out = np.empty((2, rows), np.float32)
        self._mode()
        self.lib.df_depth_step(ctypes.byref(self.dstack), _ptr(xin), depth_idx, _ptr(self.dk), _ptr(self.dv),
                               self.cfg.rvq_depth, _ptr(self.dec_norm), _ptr(head), rows, _ptr(out))
        return out

    def generate(self, opts: O.GenerateOptions, *, teacher: Optional[np.ndarray] = None,
                 record: Optional[dict] = None) -> np.ndarray:
        """generate_tokens (decode.cpp:239-573) on the cross K/V set before:
        (F, L) fed ids.  ``record`` receives 'slices' (F, L, 2, C),
        'temporal_out' / 'frame_mean' (F, 2, D) and 'drawn' (F, L), as the
        numpy oracle's record; the temporal caches are left in tk / tv and the
        last frame's depth caches in dk / dv."""
        assert self.ck is not None and opts.num_frames <= self.F
        F, L, C, D = opts.num_frames, opts.rvq_depth, opts.codebook_size, self.cfg.d_model
        assert L == self.cfg.rvq_depth
        toks = np.zeros((F, L), np.int32)
        t = None if teacher is None else np.ascontiguousarray(teacher, dtype=np.int32).reshape(F, L)
        rec = record if record is not None else {}
        sl = rec.setdefault("slices", np.zeros((F, L, 2, C), np.float32)) if record is not None else None
        to = rec.setdefault("temporal_out", np.zeros((F, 2, D), np.float32)) if record is not None else None
        fm = rec.setdefault("frame_mean", np.zeros((F, 2, D), np.float32)) if record is not None else None
        dr = rec.setdefault("drawn", np.zeros((F, L), np.int32)) if record is not None else None
        self._mode()
        self.lib.df_generate(ctypes.byref(self.tstack), ctypes.byref(self.dstack), _ptr(self.emb),
                             _ptr(self.dec_norm), _ptr(self.lm_head), F, L, C, opts.codec_offset,
                             float(opts.guidance_weight), float(opts.temperature), int(opts.top_k),
                             int(opts.seed) & ((1 << 64) - 1), _ptr(t), _ptr(self.tk), _ptr(self.tv), self.F,
                             _ptr(self.dk), _ptr(self.dv), _ptr(self.ck), _ptr(self.cv), self.ck.shape[3],
                             _ptr(toks), _ptr(sl), _ptr(to), _ptr(fm), _ptr(dr))
        return toks
