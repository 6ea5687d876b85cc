"""Seeded synthetic Depthformer weight bundles in the reference's key layout.

Keys and shapes follow model.cpp:177-198 and modules.cpp:342-381 (Linear
weights stored (out, in), modules.h:74-76); bundles are fp32 like the
reference's (modules.cpp:50-53).  Initialisation mirrors the upstream gin
(t5_1_1_flaxformer.gin): projections N(0, 1/fan_in) with q additionally
scaled by 1/sqrt(d_kv) (T5 folds the attention scale into q; the reference
SDPA uses scale 1.0, modules.cpp:290), MLP and lm_head truncated normal
N(0, 1/fan_in) clipped at 2 sigma, embeddings N(0, 1), relative-position
tables uniform with fan_avg scaling, norm weights 1 (+ optional jitter).
Each tensor draws from its own stream (seed, crc32(name)), so a tensor's
values do not depend on generation order.
"""

from __future__ import annotations

import concurrent.futures as cf
import zlib
from typing import Dict, List, Tuple

import numpy as np


def bundle_layout(cfg) -> List[Tuple[str, Tuple[int, ...]]]:
    D, HD, F, V, H = cfg.d_model, cfg.num_heads * cfg.d_kv, cfg.d_ff, cfg.vocab_size, cfg.num_heads
    out = [("token_embedding.weight", (V, D)), ("lm_head.weight", (V, D)),
           ("encoder_norm.weight", (D,)), ("decoder_norm.weight", (D,)),
           ("temporal_rel_pos.relative_attention_bias.weight", (cfg.temporal_num_buckets, H)),
           ("depth_rel_pos.relative_attention_bias.weight", (cfg.depth_num_buckets, H))]

    def attn(p):
        out.extend([(p + ".q_proj.weight", (HD, D)), (p + ".k_proj.weight", (HD, D)),
                    (p + ".v_proj.weight", (HD, D)), (p + ".o_proj.weight", (D, HD))])

    def ffn(p):
        out.extend([(p + ".wi_0.weight", (F, D)), (p + ".wi_1.weight", (F, D)),
                    (p + ".wo.weight", (D, F))])

    for i in range(cfg.num_encoder_layers):
        p = f"encoder_layers.{i}"
        out.append((p + ".pre_attn_norm.weight", (D,)))
        attn(p + ".self_attn")
        out.append((p + ".pre_ffn_norm.weight", (D,)))
        ffn(p + ".ffn")
    for i in range(cfg.num_temporal_layers):
        p = f"temporal_layers.{i}"
        out.append((p + ".pre_self_attn_norm.weight", (D,)))
        attn(p + ".self_attn")
        out.append((p + ".pre_cross_attn_norm.weight", (D,)))
        attn(p + ".cross_attn")
        out.append((p + ".pre_ffn_norm.weight", (D,)))
        ffn(p + ".ffn")
    for i in range(cfg.num_depth_layers):
        p = f"depth_layers.{i}"
        out.append((p + ".pre_self_attn_norm.weight", (D,)))
        attn(p + ".self_attn")
        out.append((p + ".pre_ffn_norm.weight", (D,)))
        ffn(p + ".ffn")
    return out


def _one(name: str, shape, seed: int, d_kv: int, norm_jitter: float) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed, zlib.crc32(name.encode())])))
    n = int(np.prod(shape))
    if name.endswith("norm.weight"):
        w = np.ones(n, dtype=np.float32)
        if norm_jitter:
            w += np.float32(norm_jitter) * rng.standard_normal(n, dtype=np.float32)
        return w.reshape(shape)
    if name == "token_embedding.weight":
        return rng.standard_normal(n, dtype=np.float32).reshape(shape)
    if "relative_attention_bias" in name:
        fan_avg = (shape[0] + shape[1]) / 2.0
        lim = np.float32(np.sqrt(3.0 / fan_avg))
        return rng.uniform(-lim, lim, n).astype(np.float32).reshape(shape)
    fan_in = shape[1]
    std = np.float32(1.0 / np.sqrt(fan_in))
    w = rng.standard_normal(n, dtype=np.float32)
    if ".wi_" in name or ".wo.weight" in name or name == "lm_head.weight":
        np.clip(w, -2.0, 2.0, out=w)
    w *= std
    if name.endswith("q_proj.weight"):
        w *= np.float32(1.0 / np.sqrt(d_kv))
    return w.reshape(shape)


def make_weights(cfg, seed: int = 1234, norm_jitter: float = 0.0, threads: int = 8) -> Dict[str, np.ndarray]:
    layout = bundle_layout(cfg)
    with cf.ThreadPoolExecutor(max_workers=threads) as ex:
        arrs = list(ex.map(lambda ks: _one(ks[0], ks[1], seed, cfg.d_kv, norm_jitter), layout))
    return {k: a for (k, _), a in zip(layout, arrs)}


def write_bundle(path, weights: Dict[str, np.ndarray]) -> None:
    """Write an fp32 ``.safetensors`` bundle."""
    from safetensors.numpy import save_file  # noqa: PLC0415
    save_file({k: np.ascontiguousarray(v, dtype=np.float32) for k, v in weights.items()}, str(path))
