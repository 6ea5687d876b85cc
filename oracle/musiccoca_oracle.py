"""CPU restatement (numpy) of the reference's MusicCoCa text path and the
style-token glue: prompt ids -> 768-dim style embedding -> 12 RVQ tokens ->
LLM-vocabulary style ids.

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module: it is
the checker the HIP text encoder is compared against.  Only ``tests/`` and
``bench.py``'s CPU baseline leg may import it.

Reference files (paths relative to ``src/magenta_realtime_mlx/``):
  * softplus                       musiccoca.cpp:46-56
  * LayerNorm (eps 1e-5, fp32)     musiccoca.cpp:62-79
  * Linear (x W^T + b)             musiccoca.cpp:85-98
  * Embedding                      musiccoca.cpp:104-112
  * CoCaMHA                        musiccoca.cpp:118-177 (scale 1/sqrt(d_head),
                                   tanh logit cap, additive mask, per-dim
                                   query scale softplus(v) / ln 2)
  * TransformerLayer               musiccoca.cpp:183-206 (pre-norm, exact GELU
                                   nn_ops.h:41-53)
  * AttentionPooler                musiccoca.cpp:212-231 (no mask)
  * MusicCoCaEncoder::embed_text   musiccoca.cpp:272-294 (x * sqrt(d_model),
                                   padding -> -1e9 additive key mask)
  * StyleModel::tokenize_text_ids  style_model.cpp:52-74 (BOS 1, pad to 128)
  * rvq_quantization               rvq.cpp:24-62 (dists = |r|^2 - 2 r.c + |c|^2,
                                   argmin, first minimum)
  * StyleModel::style_tokens_lm    style_model.cpp:106-121 + rvq_to_llm
                                   (rvq.cpp:98-103)
The SentencePiece tokenizer (the vocabulary file) is not restated: ids come in.

How each part is pinned (tests/test_oracle_musiccoca.py): LayerNorm and
softmax attention against torch (float64); GELU against math.erf; softplus
closed form; the attention core against brute-force loops; rvq_quantization
against a brute-force argmin and a round trip (sums of well-separated codebook
rows are quantised back to their indices with zero residual).
Parity unpinned: MLX's fp32 accumulation order (compared within a
tolerance; token ids exactly, away from near-ties of the argmin).
"""

from __future__ import annotations

import dataclasses
import math
from typing import Dict, Optional

import numpy as np


@dataclasses.dataclass(frozen=True)
class CocaConfig:
    """MusicCoCaConfig (musiccoca.h:151-162) + StyleModel constants
    (style_model.h:24-27); the audio-path fields are not used here."""

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


def softplus(x):
    """musiccoca.cpp:46-56: max(x, 0) + log1p(exp(-|x|))."""
    return np.maximum(x, 0) + np.log1p(np.exp(-np.abs(x)))


def gelu(x):
    """nn_ops.h:41-53: x * 0.5 * (1 + erf(x / sqrt(2)))."""
    from scipy.special import erf
    return (x * 0.5 * (1.0 + erf(x * 0.7071067811865475))).astype(x.dtype)


def layer_norm(x, w, b, eps=1e-5):
    """musiccoca.cpp:71-79."""
    mean = x.mean(axis=-1, keepdims=True)
    c = x - mean
    var = (c * c).mean(axis=-1, keepdims=True)
    return (c / np.sqrt(var + x.dtype.type(eps))) * w + b


def linear(x, w, b):
    """musiccoca.cpp:95-98: stored (out, in)."""
    return x @ w.T + b


def mha(query, key, value, p: Dict[str, np.ndarray], prefix: str, H: int, D: int, cap: float = 0.0,
        mask: Optional[np.ndarray] = None, per_dim_scale: bool = False):
    """CoCaMHA::operator() (musiccoca.cpp:138-177) for one batch element:
    query (Sq, d), key / value (Sk, d) -> (Sq, d)."""
    q = linear(query, p[prefix + ".q_proj.weight"], p[prefix + ".q_proj.bias"])
    k = linear(key, p[prefix + ".k_proj.weight"], p[prefix + ".k_proj.bias"])
    v = linear(value, p[prefix + ".v_proj.weight"], p[prefix + ".v_proj.bias"])
    Sq, Sk = q.shape[0], k.shape[0]
    q = q.reshape(Sq, H, D).transpose(1, 0, 2)
    k = k.reshape(Sk, H, D).transpose(1, 0, 2)
    v = v.reshape(Sk, H, D).transpose(1, 0, 2)
    dt = q.dtype.type
    if per_dim_scale:
        q = q * (softplus(p[prefix + "._per_dim_scale"]) / dt(math.log(2.0)))
    att = (q @ k.transpose(0, 2, 1)) * dt(1.0 / math.sqrt(D))
    if cap > 0:
        att = dt(cap) * np.tanh(att / dt(cap))
    if mask is not None:
        att = att + mask[None, None, :]
    att = att - att.max(axis=-1, keepdims=True)
    e = np.exp(att)
    att = e / e.sum(axis=-1, keepdims=True)
    out = (att @ v).transpose(1, 0, 2).reshape(Sq, H * D)
    return linear(out, p[prefix + ".o_proj.weight"], p[prefix + ".o_proj.bias"])


class OracleCoca:
    """MusicCoCaEncoder text path + StyleModel glue.  ``mode``: "fp32" (the
    reference's StyleModel dtype default) or "fp64"."""

    def __init__(self, weights: Dict[str, np.ndarray], cfg: CocaConfig, mode: str = "fp32"):
        self.cfg = cfg
        self.dt = np.float32 if mode == "fp32" else np.float64
        self.w = {k: np.asarray(v, dtype=self.dt) for k, v in weights.items()}

    def layer(self, i, x, mask):
        """TransformerLayer (musiccoca.cpp:197-206)."""
        c, w, p = self.cfg, self.w, f"text_layers.{i}"
        h = layer_norm(x, w[p + ".attn_ln.weight"], w[p + ".attn_ln.bias"])
        h = mha(h, h, h, w, p + ".attn", c.num_heads, c.d_head, cap=50.0, mask=mask)
        y = x + h
        h = layer_norm(y, w[p + ".ffn_ln.weight"], w[p + ".ffn_ln.bias"])
        h = gelu(linear(h, w[p + ".ffn_w1.weight"], w[p + ".ffn_w1.bias"]))
        h = linear(h, w[p + ".ffn_w2.weight"], w[p + ".ffn_w2.bias"])
        return y + h

    def embed_text(self, ids: np.ndarray, padding: np.ndarray, record: Optional[Dict] = None) -> np.ndarray:
        """musiccoca.cpp:272-294 for one prompt: ids (L,), padding (L,) 1.0 =
        padded -> (d_model,)."""
        c, w = self.cfg, self.w
        x = w["token_embedding.weight"][np.asarray(ids)] * self.dt(math.sqrt(c.d_model))
        mask = np.asarray(padding, dtype=self.dt) * self.dt(-1e9)
        for i in range(c.num_layers):
            x = self.layer(i, x, mask)
            if record is not None:
                record[f"layer{i}"] = x.copy()
        x = layer_norm(x, w["text_exit_ln.weight"], w["text_exit_ln.bias"])
        # AttentionPooler (musiccoca.cpp:225-231): learned query, no mask
        q = w["text_pooler.query"].reshape(1, c.d_model)
        n = layer_norm(x, w["text_pooler.ln.weight"], w["text_pooler.ln.bias"])
        out = mha(q, n, n, w, "text_pooler.attn", c.num_heads, c.pooler_d_head, per_dim_scale=True)
        return out[0]

    def tokenize(self, emb: np.ndarray) -> np.ndarray:
        return rvq_quantization(emb[None].astype(np.float32), self.w["codebooks"].astype(np.float32))[0][0]

    def style_tokens_lm(self, ids, padding, style_depth: int, codebook: int, offset: int) -> np.ndarray:
        """style_model.cpp:106-121."""
        tok = self.tokenize(self.embed_text(ids, padding))[:style_depth]
        return (offset + codebook * np.arange(style_depth) + tok).astype(np.int32)


def text_ids(raw_ids, max_len: int = 128):
    """style_model.cpp:52-74: BOS (1), then up to max_len - 1 ids, zero-padded;
    padding 1.0 where padded."""
    keep = min(len(raw_ids), max_len - 1)
    ids = np.zeros(max_len, np.int32)
    pad = np.ones(max_len, np.float32)
    ids[0] = 1
    pad[0] = 0
    ids[1:keep + 1] = np.asarray(raw_ids[:keep], dtype=np.int32)
    pad[1:keep + 1] = 0
    return ids, pad


def rvq_quantization(vectors: np.ndarray, codebooks: np.ndarray):
    """rvq.cpp:24-62: per level, dists = (|r|^2 - 2 r.c) + |c|^2 in fp32,
    token = first argmin, residual -= codebook row.  Returns (tokens (N, K),
    residual (N, D))."""
    if codebooks.ndim != 3:
        raise ValueError("rvq_quantization: codebooks must be (K, C, D)")
    if vectors.ndim != 2:
        raise ValueError("rvq_quantization: vectors must be (N, D)")
    if vectors.shape[1] != codebooks.shape[2]:
        raise ValueError("rvq_quantization: vector dim mismatches codebook dim")
    r = vectors.astype(np.float32)
    toks = []
    for k in range(codebooks.shape[0]):
        cb = codebooks[k].astype(np.float32)
        r2 = (r * r).sum(axis=-1, keepdims=True)
        c2 = (cb * cb).sum(axis=-1)
        d = (r2 - np.float32(2.0) * (r @ cb.T)) + c2
        t = np.argmin(d, axis=-1).astype(np.int32)
        toks.append(t)
        r = r - cb[t]
    return np.stack(toks, axis=-1), r
