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
import dataclasses
import math
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


# ---------------------------------------------------------------------------
# SpectroStream codec bundles (decoder + codebooks)


@dataclasses.dataclass(frozen=True)
class CodecBlock:
    in_ch: int
    out_ch: int
    stride: Tuple[int, int]
    transpose_kernel: Tuple[int, int]
    post_kernel: Tuple[int, int]


@dataclasses.dataclass(frozen=True)
class CodecShape:
    """The SpectroStream decoder's shape (spectrostream.cpp:328-362): input
    projection E -> P -> P, unfold 5, seven transposed-conv blocks, a 7x7
    output conv to (real, imag).  ``tiny()`` divides the channels by 4 and
    keeps every stride, kernel and crop (test-only)."""

    embedding_dim: int = 256
    proj_ch: int = 2560
    unfold: int = 5
    blocks: Tuple[CodecBlock, ...] = (
        CodecBlock(512, 1024, (2, 1), (4, 3), (3, 3)),
        CodecBlock(512, 256, (2, 2), (4, 4), (3, 3)),
        CodecBlock(256, 256, (1, 2), (3, 4), (3, 3)),
        CodecBlock(256, 256, (1, 2), (3, 4), (3, 3)),
        CodecBlock(256, 128, (1, 3), (3, 6), (3, 3)),
        CodecBlock(128, 128, (1, 2), (3, 4), (3, 3)),
        CodecBlock(128, 64, (1, 2), (3, 4), (3, 3)),
    )
    out_ch: int = 2
    out_kernel: Tuple[int, int] = (7, 7)
    temporal_pad: int = 1
    temporal_crop: int = 4
    n_fft: int = 960

    @property
    def input_conv_ch(self) -> int:
        return self.proj_ch // self.unfold

    @staticmethod
    def reference() -> "CodecShape":
        return CodecShape()

    @staticmethod
    def tiny() -> "CodecShape":
        r = CodecShape()
        return dataclasses.replace(r, embedding_dim=64, proj_ch=640,
                                   blocks=tuple(dataclasses.replace(b, in_ch=b.in_ch // 4, out_ch=b.out_ch // 4)
                                                for b in r.blocks))

    def channels(self):
        """The ``channels`` argument of ``mrt_df.Codec``."""
        return (self.embedding_dim, self.proj_ch, [b.in_ch for b in self.blocks], [b.out_ch for b in self.blocks])


def codec_layout(shape) -> List[Tuple[str, Tuple[int, ...]]]:
    """Decoder bundle keys and stored shapes (spectrostream.cpp:125-158,
    163-262, 356-362): conv (out, in, kH, kW), transposed conv (in, out, kH,
    kW), biases (out,)."""
    E, P, C0 = shape.embedding_dim, shape.proj_ch, shape.proj_ch // shape.unfold
    out: List[Tuple[str, Tuple[int, ...]]] = []

    def conv(name, o, i, kh, kw):
        out.append((name + ".weight", (o, i, kh, kw)))
        out.append((name + ".bias", (o,)))

    conv("input_proj.conv1", P, E, 1, 1)
    conv("input_proj.conv2", P, P, 1, 1)
    conv("input_proj.shortcut", P, E, 1, 1)
    conv("input_conv.conv1", C0, C0, 3, 3)
    conv("input_conv.conv2", C0, C0, 3, 3)
    for i, b in enumerate(shape.blocks):
        p = f"decoder_blocks.{i}"
        out.append((p + ".conv_transpose.weight", (b.in_ch, b.out_ch) + tuple(b.transpose_kernel)))
        out.append((p + ".conv_transpose.bias", (b.out_ch,)))
        conv(p + ".conv", b.out_ch, b.out_ch, *b.post_kernel)
        if b.in_ch != b.out_ch:
            conv(p + ".shortcut", b.out_ch, b.in_ch, 1, 1)
    conv("output_conv", shape.out_ch, shape.blocks[-1].out_ch, *shape.out_kernel)
    return out


def make_codec_weights(shape, seed: int = 5, levels: int = 16, codebook: int = 1024,
                       cb_std: float = 0.25) -> Dict[str, np.ndarray]:
    """Seeded fp32 decoder weights in the stored layouts plus "codebooks"
    (levels, codebook, E): conv weights N(0, 1/fan_in) (fan_in = in * kH *
    kW), biases N(0, 0.02^2), codebooks N(0, cb_std^2); each tensor from its
    own (seed, crc32(name)) stream."""
    out = {}
    for name, shp in codec_layout(shape):
        rng = np.random.default_rng([seed, zlib.crc32(name.encode())])
        if name.endswith(".bias"):
            out[name] = (0.02 * rng.standard_normal(shp)).astype(np.float32)
        else:
            fan_in = (shp[0] if ".conv_transpose." in name else shp[1]) * shp[2] * shp[3]
            out[name] = (rng.standard_normal(shp) / math.sqrt(fan_in)).astype(np.float32)
    rng = np.random.default_rng([seed, zlib.crc32(b"codebooks")])
    out["codebooks"] = (cb_std * rng.standard_normal((levels, codebook, shape.embedding_dim))).astype(np.float32)
    return out


def codec_flops(shape, frames: int) -> Dict[str, float]:
    """FLOPs (2 per multiply-add) one decode of ``frames`` RVQ frames needs:
    transposed convs over their input pixels and taps (cropped outputs
    included), block shortcuts on their input grid (a 1x1 conv commutes with
    the residual's repeat), the output conv on the rows kept after the crop,
    the iSTFT as a real DFT product."""
    fl = {}
    H, E, P = frames + shape.temporal_pad, shape.embedding_dim, shape.proj_ch
    fl["input_proj"] = 2.0 * H * (E * P + P * P + E * P)
    W, C = shape.unfold, shape.proj_ch // shape.unfold
    fl["input_conv"] = 2.0 * 2 * H * W * 9 * C * C
    n = 1
    for i, b in enumerate(shape.blocks):
        if i == 1:
            n = 2
        kh, kw = b.transpose_kernel
        sh, sw = b.stride
        t = 2.0 * n * H * W * kh * kw * b.in_ch * b.out_ch
        Ho, Wo = H * sh, W * sw
        c = 2.0 * n * Ho * Wo * b.post_kernel[0] * b.post_kernel[1] * b.out_ch * b.out_ch
        s = 2.0 * n * H * W * b.in_ch * b.out_ch if b.in_ch != b.out_ch else 0.0  # on the input grid
        fl[f"block{i}"] = t + c + s
        H, W = Ho, Wo
    fl["output_conv"] = 2.0 * n * (H - shape.temporal_crop) * W * 49 * shape.blocks[-1].out_ch * shape.out_ch
    fl["istft"] = 2.0 * 2 * (H - shape.temporal_crop) * shape.n_fft * shape.n_fft
    fl["total"] = sum(fl.values())
    return fl


# ---------------------------------------------------------------------------
# MusicCoCa text encoder bundles (text path + pooler + RVQ codebooks)


def coca_layout(cfg) -> List[Tuple[str, Tuple[int, ...]]]:
    """Text-path keys and stored shapes of the MusicCoCa bundle
    (musiccoca.cpp:183-193, 212-218, 251-266): Linear weights (out, in)."""
    D, F, HD, PD = cfg.d_model, cfg.d_ff, cfg.num_heads * cfg.d_head, cfg.num_heads * cfg.pooler_d_head
    out: List[Tuple[str, Tuple[int, ...]]] = [("token_embedding.weight", (cfg.vocab_size, D))]

    def lin(name, o, i):
        out.append((name + ".weight", (o, i)))
        out.append((name + ".bias", (o,)))

    def ln(name):
        out.append((name + ".weight", (D,)))
        out.append((name + ".bias", (D,)))

    for i in range(cfg.num_layers):
        p = f"text_layers.{i}"
        ln(p + ".attn_ln")
        lin(p + ".attn.q_proj", HD, D)
        lin(p + ".attn.k_proj", HD, D)
        lin(p + ".attn.v_proj", HD, D)
        lin(p + ".attn.o_proj", D, HD)
        ln(p + ".ffn_ln")
        lin(p + ".ffn_w1", F, D)
        lin(p + ".ffn_w2", D, F)
    ln("text_exit_ln")
    out.append(("text_pooler.query", (1, 1, D)))
    ln("text_pooler.ln")
    lin("text_pooler.attn.q_proj", PD, D)
    lin("text_pooler.attn.k_proj", PD, D)
    lin("text_pooler.attn.v_proj", PD, D)
    lin("text_pooler.attn.o_proj", D, PD)
    out.append(("text_pooler.attn._per_dim_scale", (cfg.pooler_d_head,)))
    return out


def make_coca_weights(cfg, seed: int = 9, cb_std: float = 0.05) -> Dict[str, np.ndarray]:
    """Seeded fp32 MusicCoCa text weights plus "codebooks" (rvq_depth,
    codebook_size, d_model): embeddings N(0, 1/d_model) (the encoder scales
    them by sqrt(d_model)), Linear weights N(0, 1/fan_in), biases N(0, 0.02^2),
    LayerNorm weights 1 + N(0, 0.1^2), the pooler query N(0, 1), the per-dim
    scale N(0, 0.1^2), codebooks N(0, cb_std^2)."""
    out = {}
    for name, shp in coca_layout(cfg):
        rng = np.random.default_rng([seed, zlib.crc32(name.encode())])
        if name == "token_embedding.weight":
            w = rng.standard_normal(shp, dtype=np.float32) / np.float32(math.sqrt(cfg.d_model))
        elif name.endswith("_ln.weight") or name.endswith(".ln.weight"):
            w = 1.0 + 0.1 * rng.standard_normal(shp)
        elif name.endswith(".bias"):
            w = 0.02 * rng.standard_normal(shp)
        elif name == "text_pooler.query":
            w = rng.standard_normal(shp)
        elif name.endswith("_per_dim_scale"):
            w = 0.1 * rng.standard_normal(shp)
        else:
            w = rng.standard_normal(shp) / math.sqrt(shp[1])
        out[name] = np.asarray(w, dtype=np.float32)
    rng = np.random.default_rng([seed, zlib.crc32(b"codebooks")])
    out["codebooks"] = (cb_std * rng.standard_normal((cfg.rvq_depth, cfg.codebook_size, cfg.d_model))).astype(
        np.float32)
    return out


def coca_flops(cfg) -> float:
    """FLOPs (2 per multiply-add) of one MusicCoCa embed_text (max_text_len
    rows): the text layers' projections and attention, the pooler."""
    L, D, F = cfg.max_text_len, cfg.d_model, cfg.d_ff
    HD, PD = cfg.num_heads * cfg.d_head, cfg.num_heads * cfg.pooler_d_head
    per_layer = 2.0 * L * (3 * D * HD + HD * D + 2 * D * F) + 2.0 * 2 * L * L * HD
    pooler = 2.0 * (D * PD + L * 2 * D * PD + PD * D) + 2.0 * 2 * L * PD
    return cfg.num_layers * per_layer + pooler
