"""ctypes wrapper of df_cpu.c, the C/OpenMP restatement of the decode steps.

TEST INFRASTRUCTURE ONLY: checked against the numpy oracle in
tests/test_oracle_c.py and timed as the CPU baseline by bench.py.  ``build()``
compiles ``oracle/libdf_cpu.so`` with gcc (OpenMP, AVX2/FMA code generation).
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
    cmd = ["gcc", "-O3", "-march=x86-64-v3", "-fopenmp", "-shared", "-fPIC", "-Wall", str(SRC), "-o",
           str(LIB) + ".tmp", "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"df_cpu build failed:\n{' '.join(cmd)}\n{r.stderr}")
    pathlib.Path(str(LIB) + ".tmp").replace(LIB)
    return LIB


class _Stack(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("L", "D", "HD", "H", "F", "cross")] + \
               [(n, ctypes.c_void_p) for n in ("norm_sa", "wq", "wk", "wv", "wo", "norm_ca", "cq", "co",
                                               "norm_ff", "wi0", "wi1", "wo2", "bias_tab", "buckets")]


_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists() or LIB.stat().st_mtime < SRC.stat().st_mtime:
            build()
        lib = ctypes.CDLL(str(LIB))
        p, i = ctypes.c_void_p, ctypes.c_int
        lib.df_set_threads.argtypes = [i]
        lib.df_max_threads.restype = i
        lib.df_temporal_step.argtypes = [ctypes.POINTER(_Stack), p, i, p, p, i, p, p, i, p]
        lib.df_depth_step.argtypes = [ctypes.POINTER(_Stack), p, i, p, p, i, p, p, i, p]
        _lib = lib
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


class CpuDepthformer:
    """fp32 decode steps of a Depthformer bundle (the oracle's weight dict)."""

    def __init__(self, weights: Dict[str, np.ndarray], cfg: O.DepthformerConfig, max_frames: int = 50):
        self.lib = load()
        self.cfg = cfg
        f32 = lambda k: np.ascontiguousarray(weights[k], dtype=np.float32)
        self.keep = []

        def stack(family, n, cross):
            def st(key):
                a = np.ascontiguousarray(np.stack([f32(f"{family}.{i}.{key}.weight") for i in range(n)]))
                self.keep.append(a)
                return _ptr(a)
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
        self.F = max_frames
        H = cfg.num_heads
        self.tk = np.zeros((cfg.num_temporal_layers, 2, H, max_frames, 64), np.float32)
        self.tv = np.zeros_like(self.tk)
        self.dk = np.zeros((cfg.num_depth_layers, 2, H, cfg.rvq_depth, 64), np.float32)
        self.dv = np.zeros_like(self.dk)
        self.ck: Optional[np.ndarray] = None
        self.cv: Optional[np.ndarray] = None

    @staticmethod
    def set_threads(n: int) -> None:
        load().df_set_threads(int(n))

    def set_cross(self, cross_kv) -> None:
        """cross K/V of every temporal layer: the oracle's precompute_cross_kv
        output, a list of (k, v) of shape (2, H, S, 64)."""
        self.ck = np.ascontiguousarray(np.stack([k for k, _ in cross_kv]), dtype=np.float32)
        self.cv = np.ascontiguousarray(np.stack([v for _, v in cross_kv]), dtype=np.float32)

    def temporal_step(self, x: np.ndarray, frame_idx: int) -> np.ndarray:
        assert self.ck is not None and 0 <= frame_idx < self.F
        xin = np.ascontiguousarray(x, dtype=np.float32).reshape(2, self.cfg.d_model)
        out = np.empty_like(xin)
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
        self.lib.df_depth_step(ctypes.byref(self.dstack), _ptr(xin), depth_idx, _ptr(self.dk), _ptr(self.dv),
                               self.cfg.rvq_depth, _ptr(self.dec_norm), _ptr(head), rows, _ptr(out))
        return out
