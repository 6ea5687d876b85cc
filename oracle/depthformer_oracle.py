"""CPU restatement (numpy) of the reference Depthformer streaming-decode path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module: it is the
checker that the HIP library is compared against, and the timed CPU baseline in
``bench.py``.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it.

Every function cites the reference file:line it restates (paths relative to the
reference repository root, ``src/magenta_realtime_mlx/...`` abbreviated to the
file name where unambiguous).

Precision modes (``mode``):
  * ``"fp64"`` -- everything in float64 (the mathematical truth at this input).
  * ``"fp32"`` -- float32 storage and arithmetic, like the reference with
    ``--dtype fp32``.
  * ``"bf16"`` -- bf16-emulating: values are held in float32 arrays but every
    op output the reference materialises in the model dtype is rounded to bf16
    (round-to-nearest-even), mirroring MLX's per-op bf16 outputs.  Matmul and
    softmax accumulate in float32 as MLX does.
  * ``"fp16"`` -- the same with IEEE binary16 rounding (numpy's float16 cast:
    ties to even, subnormals kept, overflow to inf), like ``--dtype fp16``
    (dtype.cpp:40-41).

How each part is pinned (see tests/test_oracle_*.py):
  * relative_position_bucket        -- closed form (identity below num_buckets/2)
                                       and brute-force Python loop.
  * sinusoidal_position_embedding   -- closed form in float64.
  * gelu_approx, rms_norm, sdpa     -- textbook formulas in float64 loops.
  * layer / step math               -- brute-force pure-Python loops at tiny
                                       dims (tests/test_oracle_bruteforce.py).
  * step chain                      -- invariant: cached depth_step logits equal
                                       depth_forward_full causal logits;
                                       temporal cached steps equal a full causal
                                       pass (upstream modules_test.py:370-416).
  * frame-mean feedback             -- invariant: temporal input equals the mean
                                       of the frame's 16 level embeddings
                                       (upstream modules_test.py:293-359).
  * sampling                        -- Philox known-answer vectors, chi-square of
                                       draws against softmax(top-k(CFG/T)).
Parity unpinned (no executable MLX here): MLX's exact bf16 rounding and
accumulation order inside fast::rms_norm / SDPA / matmul; the MLX random stream.
"""

from __future__ import annotations

import dataclasses
import math
from typing import Callable, Dict, List, Optional, Sequence, Tuple

import numpy as np

# ---------------------------------------------------------------------------
# Configuration -- model.h:47-68, model.cpp:34-48
# ---------------------------------------------------------------------------


@dataclasses.dataclass(frozen=True)
class DepthformerConfig:
    """Mirror of ``DepthformerConfig`` (model.h:47-68)."""

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
    def base() -> "DepthformerConfig":  # model.cpp:34-36
        return DepthformerConfig()

    @staticmethod
    def large() -> "DepthformerConfig":  # model.cpp:38-48
        return DepthformerConfig(d_model=1024, d_kv=64, d_ff=2816, num_heads=16,
                                 num_encoder_layers=24, num_temporal_layers=40,
                                 num_depth_layers=8)

    @staticmethod
    def bench() -> "DepthformerConfig":
        """d_model 1024 / 16 heads / d_ff 2816 with 12/20/4 layers."""
        return DepthformerConfig(d_model=1024, d_kv=64, d_ff=2816, num_heads=16,
                                 num_encoder_layers=12, num_temporal_layers=20,
                                 num_depth_layers=4)

    @staticmethod
    def tiny(codebook: int = 8) -> "DepthformerConfig":
        """Small model for golden vectors: 16 levels of ``codebook`` codes, head dim 64."""
        return DepthformerConfig(vocab_size=2 + 16 * codebook + 6 * codebook,
                                 d_model=128, d_kv=64, d_ff=192, num_heads=2,
                                 num_encoder_layers=2, num_temporal_layers=2,
                                 num_depth_layers=2, max_encoder_length=46,
                                 rvq_depth=16, temporal_num_buckets=128,
                                 temporal_max_distance=128, depth_num_buckets=16,
                                 depth_max_distance=16)


# ---------------------------------------------------------------------------
# Precision helpers
# ---------------------------------------------------------------------------


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even); float32 out."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).reshape(a.shape)
    nan = np.isnan(a)
    if nan.any():
        out = np.where(nan, np.float32(np.nan), out)
    return out


def round_fp16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest binary16 (ties to even); float32 out."""
    with np.errstate(over="ignore"):
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


class Precision:
    """Storage/compute precision of the restatement (see module docstring)."""

    def __init__(self, mode: str):
        if mode not in ("fp64", "fp32", "bf16", "fp16"):
            raise ValueError(f"unknown mode {mode!r}")
        self.mode = mode
        self.dtype = np.float64 if mode == "fp64" else np.float32

    def r(self, x) -> np.ndarray:
        """Materialise ``x`` in the model dtype (an MLX op output)."""
        x = np.asarray(x, dtype=self.dtype)
        if self.mode == "bf16":
            return round_bf16(x)
        if self.mode == "fp16":
            return round_fp16(x)
        return x

    def c(self, v: float):
        """A scalar literal cast to the model dtype (nn_ops.h:76-79)."""
        return self.r(np.array(v, dtype=np.float32))


# ---------------------------------------------------------------------------
# Relative position bias -- modules.cpp:139-191, model.cpp:302-320
# ---------------------------------------------------------------------------


def relative_position_bucket(relative_position: np.ndarray, bidirectional: bool,
                             num_buckets: int, max_distance: int) -> np.ndarray:
    """T5 bucketing restated from modules.cpp:139-174 (float32 log branch)."""
    rel = np.asarray(relative_position, dtype=np.int32)
    eff = num_buckets
    ret = np.zeros(rel.shape, dtype=np.int32)
    n = -rel
    if bidirectional:
        eff //= 2
        ret = ret + np.where(n < 0, eff, 0).astype(np.int32)
        n = np.abs(n)
    else:
        n = np.maximum(n, 0)
    max_exact = eff // 2
    is_small = n < max_exact
    log_ratio = np.float32(math.log(np.float32(max_distance) / np.float32(max_exact)))
    with np.errstate(divide="ignore", invalid="ignore"):
        nf = n.astype(np.float32)
        lg = np.log(nf / np.float32(max_exact)).astype(np.float32)
        large_f = (np.float32(max_exact)
                   + (lg / log_ratio).astype(np.float32) * np.float32(eff - max_exact))
        large_f = np.where(np.isfinite(large_f), large_f, 0).astype(np.float32)
    val_if_large = np.trunc(large_f).astype(np.int32)
    val_if_large = np.minimum(val_if_large, eff - 1)
    return (ret + np.where(is_small, n, val_if_large)).astype(np.int32)


def rel_pos_bias(table: np.ndarray, query_length: int, key_length: int,
                 offset: int, num_buckets: int, max_distance: int) -> np.ndarray:
    """``RelativePositionBias::operator()`` (modules.cpp:178-191) -> (1,H,Q,K)."""
    ctx = np.arange(offset, offset + query_length, dtype=np.int32)
    mem = np.arange(0, key_length, dtype=np.int32)
    rel = mem[None, :] - ctx[:, None]
    buckets = relative_position_bucket(rel, False, num_buckets, max_distance)
    values = table[buckets]                      # (Q, K, H)
    return np.transpose(values, (2, 0, 1))[None]  # (1, H, Q, K)


# ---------------------------------------------------------------------------
# Sinusoidal position embedding -- model.cpp:54-80
# ---------------------------------------------------------------------------


def sinusoidal_position_embedding(max_length: int, features: int,
                                  min_scale: float = 1.0,
                                  max_scale: float = 10000.0) -> np.ndarray:
    """float32 table, restating model.cpp:54-80 op for op in float32."""
    half = features // 2
    if half <= 1:
        raise RuntimeError("features // 2 must be >= 2 for sinusoidal PE")
    f32 = np.float32
    scale_factor = f32(-np.log(f32(max_scale) / f32(min_scale))) / f32(half - 1)
    div_term = f32(min_scale) * np.exp(np.arange(half, dtype=np.float32) * scale_factor)
    pos = np.arange(max_length, dtype=np.float32)[:, None]
    angle = (pos * div_term[None, :]).astype(np.float32)
    out = np.zeros((max_length, features), dtype=np.float32)
    out[:, :half] = np.sin(angle)
    out[:, half:2 * half] = np.cos(angle)
    return out


# ---------------------------------------------------------------------------
# Elementwise ops -- nn_ops.h:66-98, modules.cpp:72-84
# ---------------------------------------------------------------------------


def gelu_approx(x: np.ndarray, P: Precision) -> np.ndarray:
    """Tanh GELU with per-op rounding to the model dtype (nn_ops.h:66-84)."""
    half, one = P.c(0.5), P.c(1.0)
    c0, c1 = P.c(0.7978845608028654), P.c(0.044715)
    x2 = P.r(x * x)
    t = P.r(c1 * x2)
    t = P.r(one + t)
    t = P.r(x * t)
    inner = P.r(c0 * t)
    th = P.r(np.tanh(inner))
    t = P.r(one + th)
    t = P.r(x * t)
    return P.r(half * t)


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float, P: Precision) -> np.ndarray:
    """``mx::fast::rms_norm`` (modules.cpp:83): x*rsqrt(mean(x^2)+eps)*w.

    Reduction in float32 (float64 in fp64 mode); the normalised value is
    materialised in the model dtype before the weight multiply.
    """
    acc_t = np.float64 if P.mode == "fp64" else np.float32
    xf = x.astype(acc_t)
    ms = np.mean(xf * xf, axis=-1, keepdims=True, dtype=acc_t)
    inv = (1.0 / np.sqrt(ms + acc_t(eps))).astype(acc_t)
    return P.r(P.r(xf * inv) * w)


def sdpa(q: np.ndarray, k: np.ndarray, v: np.ndarray,
         mask: Optional[np.ndarray], P: Precision) -> np.ndarray:
    """``mx::fast::scaled_dot_product_attention`` with scale 1.0 (modules.cpp:289-290)."""
    acc_t = np.float64 if P.mode == "fp64" else np.float32
    s = np.matmul(q.astype(acc_t), np.swapaxes(k.astype(acc_t), -1, -2))
    if mask is not None:
        s = s + mask.astype(acc_t)
    m = np.max(s, axis=-1, keepdims=True)
    e = np.exp(s - m)
    p = e / np.sum(e, axis=-1, keepdims=True)
    return P.r(np.matmul(p, v.astype(acc_t)))


def causal_mask(seq_len: int) -> np.ndarray:
    """modules.cpp:197-209: -inf strictly above the diagonal, (1,1,S,S)."""
    m = np.triu(np.full((seq_len, seq_len), -np.inf, dtype=np.float32), k=1)
    return m[None, None]


# ---------------------------------------------------------------------------
# The model -- modules.cpp:215-455, model.cpp:173-659
# ---------------------------------------------------------------------------

LayerCache = Dict[str, Optional[np.ndarray]]  # keys: k, v, ck, cv


class OracleDepthformer:
    """Numpy restatement of ``Depthformer`` (model.h:72-239)."""

    def __init__(self, weights: Dict[str, np.ndarray], cfg: DepthformerConfig,
                 mode: str = "fp32"):
        self.cfg = cfg
        self.P = Precision(mode)
        # load_param casts each fp32 bundle tensor to the compute dtype
        # (modules.cpp:47-54).
        self.w = {k: self.P.r(np.asarray(v, dtype=np.float32)) for k, v in weights.items()}
        self.eps = 1e-6  # modules.cpp:342-346, 369-374
        # model.cpp:178-179: fp32 table built at construction.
        self.pe = sinusoidal_position_embedding(cfg.max_encoder_length, cfg.d_model)

    # -- building blocks ---------------------------------------------------
    def linear(self, x: np.ndarray, key: str) -> np.ndarray:
        """Bias-free Linear, weight stored (out,in) (modules.cpp:90-100)."""
        W = self.w[key + ".weight"]
        acc_t = np.float64 if self.P.mode == "fp64" else np.float32
        return self.P.r(np.matmul(x.astype(acc_t), W.T.astype(acc_t)))

    def norm(self, x: np.ndarray, key: str) -> np.ndarray:
        return rms_norm(x, self.w[key + ".weight"], self.eps, self.P)

    def embed(self, ids: np.ndarray) -> np.ndarray:
        """Embedding gather (modules.cpp:110-112)."""
        return self.w["token_embedding.weight"][np.asarray(ids, dtype=np.int64)]

    def ffn(self, x: np.ndarray, prefix: str) -> np.ndarray:
        """GatedFeedForward (modules.cpp:222-226): wo(gelu(wi_0 x) * wi_1 x)."""
        a = self.linear(x, prefix + ".wi_0")
        b = self.linear(x, prefix + ".wi_1")
        return self.linear(self.P.r(gelu_approx(a, self.P) * b), prefix + ".wo")

    def _heads(self, y: np.ndarray) -> np.ndarray:
        """(B, T, H*D) -> (B, T, H, D) -> (B, H, T, D) (modules.cpp:251-253, 264-269)."""
        B, T, _ = y.shape
        return y.reshape(B, T, self.cfg.num_heads, self.cfg.d_kv).transpose(0, 2, 1, 3)

    def _merge_heads(self, o: np.ndarray) -> np.ndarray:
        """(B, H, T, D) -> (B, T, H, D) -> (B, T, H*D) (modules.cpp:291-293)."""
        B, _, T, _ = o.shape
        return o.transpose(0, 2, 1, 3).reshape(B, T, self.cfg.num_heads * self.cfg.d_kv)

    def mha(self, x: np.ndarray, prefix: str, *, context: Optional[np.ndarray] = None,
            mask: Optional[np.ndarray] = None, bias: Optional[np.ndarray] = None,
            past: Optional[Tuple[np.ndarray, np.ndarray]] = None,
            cross: Optional[Tuple[np.ndarray, np.ndarray]] = None):
        """MultiHeadAttention::forward (modules.cpp:243-295). Returns (out, (k, v))."""
        q = self._heads(self.linear(x, prefix + ".q_proj"))
        if cross is not None:
            k, v = cross  # modules.cpp:258-261: cached cross K/V reused verbatim
        else:
            src = x if context is None else context
            k = self._heads(self.linear(src, prefix + ".k_proj"))
            v = self._heads(self.linear(src, prefix + ".v_proj"))
            if past is not None:  # modules.cpp:271-275
                k = np.concatenate([past[0], k], axis=2)
                v = np.concatenate([past[1], v], axis=2)
        attn_mask = None
        if bias is not None and mask is not None:
            attn_mask = self.P.r(bias + mask)
        elif bias is not None:
            attn_mask = bias
        elif mask is not None:
            attn_mask = mask
        o = sdpa(q, k, v, attn_mask, self.P)
        return self.linear(self._merge_heads(o), prefix + ".o_proj"), (k, v)

    def project_kv(self, context: np.ndarray, prefix: str):
        """MultiHeadAttention::project_kv (modules.cpp:323-333)."""
        k = self._heads(self.linear(context, prefix + ".k_proj"))
        v = self._heads(self.linear(context, prefix + ".v_proj"))
        return k, v

    # -- encoder -- modules.cpp:349-358, model.cpp:226-241 ------------------
    def encoder_layer(self, x: np.ndarray, i: int) -> np.ndarray:
        p = f"encoder_layers.{i}"
        h, _ = self.mha(self.norm(x, p + ".pre_attn_norm"), p + ".self_attn")
        y = self.P.r(x + h)
        f = self.ffn(self.norm(y, p + ".pre_ffn_norm"), p + ".ffn")
        return self.P.r(y + f)

    def encode(self, tokens: np.ndarray) -> np.ndarray:
        tokens = np.asarray(tokens, dtype=np.int64)
        S = tokens.shape[1]
        if S > self.cfg.max_encoder_length:
            raise IndexError("seq_len exceeds max_encoder_length")  # model.cpp:216-218
        x = self.embed(tokens)
        pe = self.P.r(self.pe[:S])  # cast to x dtype before the add (model.cpp:232-236)
        x = self.P.r(x + pe[None])
        for i in range(self.cfg.num_encoder_layers):
            x = self.encoder_layer(x, i)
        return self.norm(x, "encoder_norm")

    # -- decoder layers -- modules.cpp:384-408 -------------------------------
    def decoder_layer(self, x: np.ndarray, family: str, i: int, *,
                      bias: Optional[np.ndarray], mask: Optional[np.ndarray] = None,
                      past: Optional[Tuple[np.ndarray, np.ndarray]] = None,
                      enc_out: Optional[np.ndarray] = None,
                      cross: Optional[Tuple[np.ndarray, np.ndarray]] = None):
        p = f"{family}.{i}"
        h, self_kv = self.mha(self.norm(x, p + ".pre_self_attn_norm"), p + ".self_attn",
                              mask=mask, bias=bias, past=past)
        y = self.P.r(x + h)
        cross_kv = None
        if family == "temporal_layers" and (enc_out is not None or cross is not None):
            h2, cross_kv = self.mha(self.norm(y, p + ".pre_cross_attn_norm"),
                                    p + ".cross_attn", context=enc_out, cross=cross)
            y = self.P.r(y + h2)
        f = self.ffn(self.norm(y, p + ".pre_ffn_norm"), p + ".ffn")
        return self.P.r(y + f), self_kv, cross_kv

    # -- caches and biases -- model.cpp:280-320 ------------------------------
    def empty_temporal_cache(self) -> List[LayerCache]:
        return [dict(k=None, v=None, ck=None, cv=None) for _ in range(self.cfg.num_temporal_layers)]

    def empty_depth_cache(self) -> List[LayerCache]:
        return [dict(k=None, v=None, ck=None, cv=None) for _ in range(self.cfg.num_depth_layers)]

    def temporal_bias(self, frame_idx: int, key_length: Optional[int] = None,
                      query_length: int = 1) -> np.ndarray:
        c = self.cfg
        kl = frame_idx + 1 if key_length is None else key_length
        return rel_pos_bias(self.w["temporal_rel_pos.relative_attention_bias.weight"],
                            query_length, kl, frame_idx, c.temporal_num_buckets,
                            c.temporal_max_distance)

    def depth_bias(self, depth_idx: int, key_length: Optional[int] = None,
                   query_length: int = 1) -> np.ndarray:
        c = self.cfg
        kl = depth_idx + 1 if key_length is None else key_length
        return rel_pos_bias(self.w["depth_rel_pos.relative_attention_bias.weight"],
                            query_length, kl, depth_idx, c.depth_num_buckets,
                            c.depth_max_distance)

    def precompute_cross_kv(self, enc_out: np.ndarray):
        """DecoderLayer::precompute_cross_kv for every temporal layer (modules.cpp:448-455)."""
        return [self.project_kv(enc_out, f"temporal_layers.{i}.cross_attn")
                for i in range(self.cfg.num_temporal_layers)]

    # -- steps -- model.cpp:322-659 -------------------------------------------
    def temporal_step(self, frame_emb: np.ndarray, enc_out: np.ndarray,
                      cache: List[LayerCache], frame_idx: int,
                      position_bias: Optional[np.ndarray] = None) -> np.ndarray:
        """Eager temporal_step (model.cpp:493-513): 20 layers, no final norm.
        position_bias (1, H, 1, frame_idx + 1) replaces the rel-pos bias (model.cpp:330-332)."""
        if len(cache) != self.cfg.num_temporal_layers:
            raise RuntimeError("temporal_step: cache size mismatch")  # model.cpp:326-328
        bias = self.temporal_bias(frame_idx) if position_bias is None else position_bias
        first = frame_idx == 0
        x = frame_emb
        for i, lc in enumerate(cache):
            past = None if first else (lc["k"], lc["v"])
            cross = None if first else (lc["ck"], lc["cv"])
            x, (k, v), ckv = self.decoder_layer(
                x, "temporal_layers", i, bias=bias, past=past,
                enc_out=enc_out if cross is None else None, cross=cross)
            lc["k"], lc["v"] = k, v
            if ckv is not None:
                lc["ck"], lc["cv"] = ckv
        return x

    def depth_step(self, tok_emb: np.ndarray, cache: List[LayerCache],
                   depth_idx: int, position_bias: Optional[np.ndarray] = None) -> np.ndarray:
        """Eager depth_step (model.cpp:638-658): 4 layers + decoder_norm + lm_head.
        position_bias (1, H, 1, depth_idx + 1) replaces the rel-pos bias (model.cpp:523-525)."""
        if len(cache) != self.cfg.num_depth_layers:
            raise RuntimeError("depth_step: cache size mismatch")  # model.cpp:519-521
        bias = self.depth_bias(depth_idx) if position_bias is None else position_bias
        first = depth_idx == 0
        x = tok_emb
        for i, lc in enumerate(cache):
            past = None if first else (lc["k"], lc["v"])
            x, (k, v), _ = self.decoder_layer(x, "depth_layers", i, bias=bias, past=past)
            lc["k"], lc["v"] = k, v
        x = self.norm(x, "decoder_norm")
        logits = self.linear(x, "lm_head")
        return logits[:, 0, :]

    def depth_forward_full(self, embs: np.ndarray, causal: bool = True,
                           position_bias: Optional[np.ndarray] = None) -> np.ndarray:
        """Full-sequence depth pass (model.cpp:243-268) -> (B, K, V); position_bias
        (1, H, K, K) replaces the rel-pos block of query offset 0 (model.cpp:248-250)."""
        K = embs.shape[1]
        bias = self.depth_bias(0, key_length=K, query_length=K) if position_bias is None else position_bias
        mask = causal_mask(K) if causal else None
        if mask is not None:
            mask = self.P.r(mask)
        x = embs
        for i in range(self.cfg.num_depth_layers):
            x, _, _ = self.decoder_layer(x, "depth_layers", i, bias=bias, mask=mask)
        return self.linear(self.norm(x, "decoder_norm"), "lm_head")

    def temporal_forward_full(self, frame_embs: np.ndarray, enc_out: np.ndarray) -> np.ndarray:
        """Causal full-sequence temporal pass (invariant target for temporal_step)."""
        F = frame_embs.shape[1]
        bias = self.temporal_bias(0, key_length=F, query_length=F)
        mask = self.P.r(causal_mask(F))
        x = frame_embs
        for i in range(self.cfg.num_temporal_layers):
            x, _, _ = self.decoder_layer(x, "temporal_layers", i, bias=bias, mask=mask,
                                         enc_out=enc_out)
        return x


# ---------------------------------------------------------------------------
# Decode loop -- decode.cpp:71-148, 239-573
# ---------------------------------------------------------------------------


def cfg_combine(logits_2v: np.ndarray, guidance_weight: float) -> np.ndarray:
    """decode.cpp:71-85 / upstream decode.py:87-89: fp32 (1+w)*l0 - w*l1."""
    f32 = np.float32
    cond = logits_2v[0].astype(np.float32)
    unc = logits_2v[1].astype(np.float32)
    a = (f32(1.0 + guidance_weight) * cond).astype(np.float32)
    b = (f32(guidance_weight) * unc).astype(np.float32)
    return (a - b).astype(np.float32)


def top_k_threshold(scaled: np.ndarray, k: int) -> np.float32:
    """min(topk(x, k)) -- the k-th largest value counting ties (decode.cpp:119-120)."""
    return np.float32(np.sort(scaled)[::-1][k - 1])


def top_k_logits(scaled: np.ndarray, k: int) -> np.ndarray:
    """decode.cpp:104-122: entries strictly below the k-th largest -> -inf."""
    if k <= 0:
        return scaled
    thr = top_k_threshold(scaled, k)
    return np.where(scaled < thr, np.float32(-np.inf), scaled).astype(np.float32)


# ---- counter-based RNG (our own; the MLX stream is not reproducible here) ----

PHILOX_M0, PHILOX_M1 = 0xD2511F53, 0xCD9E8D57
PHILOX_W0, PHILOX_W1 = 0x9E3779B9, 0xBB67AE85
MASK32 = 0xFFFFFFFF


def philox4x32_10(ctr: Sequence[np.ndarray], key: Sequence[int]) -> List[np.ndarray]:
    """Philox-4x32-10 (Salmon et al., SC'11), vectorised over counters."""
    c = [np.asarray(x, dtype=np.uint64) & MASK32 for x in ctr]
    c = np.broadcast_arrays(*c)
    c = [x.copy() for x in c]
    k0, k1 = np.uint64(key[0] & MASK32), np.uint64(key[1] & MASK32)
    for r in range(10):
        if r:
            k0 = np.uint64((int(k0) + PHILOX_W0) & MASK32)
            k1 = np.uint64((int(k1) + PHILOX_W1) & MASK32)
        p0 = c[0] * np.uint64(PHILOX_M0)
        p1 = c[2] * np.uint64(PHILOX_M1)
        hi0, lo0 = p0 >> np.uint64(32), p0 & np.uint64(MASK32)
        hi1, lo1 = p1 >> np.uint64(32), p1 & np.uint64(MASK32)
        c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
    return [x.astype(np.uint32) for x in c]


SAMPLE_STREAM_TAG = 0x4D525444  # fourth Philox counter word of every draw


def gumbel_noise(seed: int, frame: int, level: int, n: int) -> np.ndarray:
    """Gumbel(0,1) noise for one draw; candidate i uses counter (i, level, frame, tag).

    u = ((x >> 9) + 0.5) * 2^-23, strictly inside (0,1);  g = -log(-log(u)) in float32.
    """
    i = np.arange(n, dtype=np.uint64)
    x = philox4x32_10([i, level, frame, SAMPLE_STREAM_TAG], [seed & MASK32, (seed >> 32) & MASK32])[0]
    u = ((x >> np.uint32(9)).astype(np.float32) + np.float32(0.5)) * np.float32(2.0 ** -23)
    return (-np.log(-np.log(u))).astype(np.float32)


def sample_level(guided_slice: np.ndarray, *, temperature: float, top_k: int,
                 seed: int, frame: int, level: int) -> int:
    """Categorical draw over one level's slice (decode.cpp:124-148).

    ``guided_slice`` is the CFG-combined fp32 logits of the level's codebook
    range.  temperature == 0 -> argmax (first max).  Otherwise
    argmax(top_k(guided / T) + gumbel), i.e. a categorical draw by Gumbel-max,
    which is how ``mx::random::categorical`` samples.
    Returns the index within the slice.
    """
    g = guided_slice.astype(np.float32)
    if temperature == 0.0:
        return int(np.argmax(g))
    scaled = (g / np.float32(temperature)).astype(np.float32)
    if top_k > 0:
        scaled = top_k_logits(scaled, min(top_k, scaled.size))
    noise = gumbel_noise(seed, frame, level, scaled.size)
    return int(np.argmax((scaled + noise).astype(np.float32)))


@dataclasses.dataclass
class GenerateOptions:
    """decode.h:48-57 (guidance 4.0 default; streaming uses 5.0, system.h:89)."""

    num_frames: int = 50
    rvq_depth: int = 16
    temperature: float = 1.1
    top_k: int = 40
    guidance_weight: float = 4.0
    seed: int = 0
    codebook_size: int = 1024
    codec_offset: int = 2


def generate_tokens(model: OracleDepthformer, enc_tokens: np.ndarray,
                    opts: GenerateOptions, *, teacher: Optional[np.ndarray] = None,
                    record: Optional[dict] = None,
                    enc_out: Optional[np.ndarray] = None) -> np.ndarray:
    """Block-autoregressive decode (decode.cpp:239-573), non-speculative path.

    ``teacher`` (F, L) LLM ids: teacher forcing (the fed-back token is the
    teacher token, the model's draw is still recorded).  ``record`` collects
    per-step data: 'slices' (F, L, 2, C) level-slice logits in model dtype,
    'temporal_out' (F, 2, D), 'frame_mean' (F, 2, D), 'drawn' (F, L) ids, and
    at the end 'temporal_cache' (every temporal layer's K/V over all frames)
    and 'depth_cache' (the last frame's depth K/V).
    Returns (F, L) int32 LLM ids (the fed-back tokens).
    """
    P = model.P
    C, off = opts.codebook_size, opts.codec_offset
    if enc_out is None:
        enc_out = model.encode(enc_tokens)
    B = enc_tokens.shape[0]
    D = model.cfg.d_model
    F, L = opts.num_frames, opts.rvq_depth
    out = np.zeros((F, L), dtype=np.int32)
    if record is not None:
        record.setdefault("slices", np.zeros((F, L, B, C), dtype=np.float32))
        record.setdefault("temporal_out", np.zeros((F, B, D), dtype=np.float32))
        record.setdefault("frame_mean", np.zeros((F, B, D), dtype=np.float32))
        record.setdefault("drawn", np.zeros((F, L), dtype=np.int32))
        record.setdefault("enc_out", enc_out)
    tcache = model.empty_temporal_cache()
    prev_mean = None
    rvq_div = P.c(float(L))  # decode.cpp:271-273: divisor in the model dtype
    for f in range(F):
        # decode.cpp:366-368: frame 0 feeds emb(PAD=0) on both rows.
        t_in = model.embed(np.zeros((B, 1), dtype=np.int64)) if f == 0 else prev_mean
        t_out = model.temporal_step(t_in, enc_out, tcache, f)
        if record is not None:
            record["temporal_out"][f] = t_out[:, 0]
        dcache = model.empty_depth_cache()
        d_in = t_out
        fsum = np.zeros((B, 1, D), dtype=P.dtype)
        for lvl in range(L):
            logits = model.depth_step(d_in, dcache, lvl)  # (B, V)
            lo = off + C * lvl
            sl = logits[:, lo:lo + C]
            guided = cfg_combine(sl, opts.guidance_weight)
            drawn = lo + sample_level(guided, temperature=opts.temperature, top_k=opts.top_k,
                                      seed=opts.seed, frame=f, level=lvl)
            tok = drawn if teacher is None else int(teacher[f, lvl])
            out[f, lvl] = tok
            if record is not None:
                record["slices"][f, lvl] = sl
                record["drawn"][f, lvl] = drawn
            # decode.cpp:476-477: both rows take the same token.
            d_in = model.embed(np.full((B, 1), tok, dtype=np.int64))
            fsum = P.r(fsum + d_in)
        prev_mean = P.r(fsum / rvq_div)  # decode.cpp:484
        if record is not None:
            record["frame_mean"][f] = prev_mean[:, 0]
            record["depth_cache"] = dcache
    if record is not None:
        record["temporal_cache"] = tcache
    return out
