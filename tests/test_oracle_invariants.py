"""Pins the oracle's layer and step math without the reference (whose MLX
implementation cannot run here): brute-force pure-Python loops at micro
dims, and the structural invariants the reference's own design relies on:

  (i)   step-by-step depth logits == the full causal depth pass
        (depth_forward_full, model.cpp:243-268; model.h:27-31; upstream
        modules_test.py:370-416);
  (ii)  step-by-step temporal outputs == the full causal temporal pass;
  (iii) cached K/V rows == K/V projections of the prefix (modules.cpp:271-275);
  (iv)  the depth cache starts empty every frame (decode.cpp:454; upstream
        modules_test.py:238-280);
  (v)   the next temporal input is the model-dtype mean of the frame's 16
        token embeddings (decode.cpp:263-273, 476-484; upstream
        modules_test.py:293-359);
  (vi)  attention over a fixed ring with -inf past the cache length equals
        attention over the concatenated prefix (model.h:219-231).
All checks run in float64 so that a wrong sign, index or operand shows up
far above rounding noise.
"""

from __future__ import annotations

import dataclasses
import math

import numpy as np
import pytest

from oracle import depthformer_oracle as O

import synth_bundle


def micro_cfg():
    # two heads of 32 with d_model 64: the brute force splits heads by hand, so a
    # transposed (T, D, H) split or a wrong bias column shows up
    return O.DepthformerConfig(vocab_size=2 + 4 * 4, d_model=64, d_kv=32, d_ff=64, num_heads=2,
                               num_encoder_layers=1, num_temporal_layers=1, num_depth_layers=1,
                               max_encoder_length=8, rvq_depth=4)


def weights_for(cfg, seed=3):
    w = synth_bundle.make_weights(cfg, seed=seed, norm_jitter=0.3)
    return {k: v.astype(np.float64) for k, v in w.items()}


@pytest.fixture(scope="module")
def micro():
    cfg = micro_cfg()
    om = O.OracleDepthformer(weights_for(cfg), cfg, mode="fp64")
    return cfg, om.w, om  # the brute force reads the weights the oracle holds


@pytest.fixture(scope="module")
def tiny():
    cfg = O.DepthformerConfig.tiny()
    om = O.OracleDepthformer(weights_for(cfg, seed=5), cfg, mode="fp64")
    return cfg, om.w, om


# ---- brute force -----------------------------------------------------------------

def b_rms(x, g, eps=1e-6):
    ms = sum(v * v for v in x) / len(x)
    inv = 1.0 / math.sqrt(ms + eps)
    return [x[i] * inv * g[i] for i in range(len(x))]


def b_lin(W, x):
    return [sum(W[j][i] * x[i] for i in range(len(x))) for j in range(len(W))]


# nn_ops.h:66-84 writes the constants as float literals: sqrt(2/pi) and 0.044715 in float32
C0 = float(np.float32(math.sqrt(2.0 / math.pi)))
C1 = float(np.float32(0.044715))


def b_gelu(x):
    return 0.5 * x * (1.0 + math.tanh(C0 * (x + C1 * x ** 3)))


def b_attend(q, keys, vals, bias):
    """One head: softmax(q.k + bias) . v, scale 1.0 (modules.cpp:289-290)."""
    s = [sum(q[d] * k[d] for d in range(len(q))) + b for k, b in zip(keys, bias)]
    m = max(s)
    e = [math.exp(v - m) for v in s]
    z = sum(e)
    return [sum(e[j] / z * vals[j][d] for j in range(len(vals))) for d in range(len(q))]


def b_mha(q, keys, vals, bias, H):
    """H heads over full-width rows.  Head h owns elements [h*D, (h+1)*D) of every
    projection row -- the (B, T, H, D) reshape of modules.cpp:251-253 -- and its
    bias is column h of the per-key bias rows (``bias[j][h]``).  The heads'
    outputs are concatenated in head order (modules.cpp:291-293)."""
    D = len(q) // H
    out = []
    for h in range(H):
        sl = slice(h * D, (h + 1) * D)
        out += b_attend(q[sl], [k[sl] for k in keys], [v[sl] for v in vals], [b[h] for b in bias])
    return out


def b_decoder_step(w, p, x, past_k, past_v, bias, H, enc=None):
    """One decoder layer for one query row; ``bias[j][h]`` is key j's bias for head h."""
    W = lambda k: w[f"{p}.{k}.weight"].tolist()
    xn = b_rms(x, w[f"{p}.pre_self_attn_norm.weight"].tolist())
    q, k, v = b_lin(W("self_attn.q_proj"), xn), b_lin(W("self_attn.k_proj"), xn), b_lin(W("self_attn.v_proj"), xn)
    o = b_mha(q, past_k + [k], past_v + [v], bias, H)
    y = [a + b for a, b in zip(x, b_lin(W("self_attn.o_proj"), o))]
    if enc is not None:
        yn = b_rms(y, w[f"{p}.pre_cross_attn_norm.weight"].tolist())
        cq = b_lin(W("cross_attn.q_proj"), yn)
        ck = [b_lin(W("cross_attn.k_proj"), e) for e in enc]
        cv = [b_lin(W("cross_attn.v_proj"), e) for e in enc]
        co = b_mha(cq, ck, cv, [[0.0] * H] * len(enc), H)
        y = [a + b for a, b in zip(y, b_lin(W("cross_attn.o_proj"), co))]
    yn = b_rms(y, w[f"{p}.pre_ffn_norm.weight"].tolist())
    g, u = b_lin(W("ffn.wi_0"), yn), b_lin(W("ffn.wi_1"), yn)
    h = [b_gelu(a) * b for a, b in zip(g, u)]
    return [a + b for a, b in zip(y, b_lin(W("ffn.wo"), h))], k, v


def test_depth_layer_bruteforce(micro):
    cfg, w, om = micro
    rng = np.random.default_rng(0)
    embs = rng.standard_normal((1, 4, cfg.d_model))
    cache = om.empty_depth_cache()
    table = w["depth_rel_pos.relative_attention_bias.weight"]
    pk, pv = [], []
    for l in range(4):
        got, (k, v), _ = om.decoder_layer(embs[:, l:l + 1], "depth_layers", 0, bias=om.depth_bias(l),
                                          past=None if l == 0 else (cache[0]["k"], cache[0]["v"]))
        cache[0]["k"], cache[0]["v"] = k, v
        bias = [table[l - j].tolist() for j in range(l + 1)]  # bucket(n) = n for n < 16
        exp, bk, bv = b_decoder_step(w, "depth_layers.0", embs[0, l].tolist(), pk, pv, bias, cfg.num_heads)
        pk.append(bk)
        pv.append(bv)
        np.testing.assert_allclose(got[0, 0], exp, rtol=1e-10, atol=1e-10)


def test_temporal_layer_bruteforce(micro):
    cfg, w, om = micro
    rng = np.random.default_rng(1)
    embs = rng.standard_normal((1, 3, cfg.d_model))
    enc = rng.standard_normal((1, 5, cfg.d_model))
    table = w["temporal_rel_pos.relative_attention_bias.weight"]
    cache = om.empty_temporal_cache()
    pk, pv = [], []
    for f in range(3):
        first = f == 0
        got, (k, v), ckv = om.decoder_layer(
            embs[:, f:f + 1], "temporal_layers", 0, bias=om.temporal_bias(f),
            past=None if first else (cache[0]["k"], cache[0]["v"]),
            enc_out=enc if first else None, cross=None if first else (cache[0]["ck"], cache[0]["cv"]))
        cache[0]["k"], cache[0]["v"] = k, v
        if ckv is not None:
            cache[0]["ck"], cache[0]["cv"] = ckv
        bias = [table[f - j].tolist() for j in range(f + 1)]
        exp, bk, bv = b_decoder_step(w, "temporal_layers.0", embs[0, f].tolist(), pk, pv, bias,
                                     cfg.num_heads, enc=enc[0].tolist())
        pk.append(bk)
        pv.append(bv)
        np.testing.assert_allclose(got[0, 0], exp, rtol=1e-10, atol=1e-10)


def test_encoder_layer_bruteforce(micro):
    cfg, w, om = micro
    rng = np.random.default_rng(2)
    x = rng.standard_normal((1, 5, cfg.d_model))
    got = om.encoder_layer(x, 0)
    p = "encoder_layers.0"
    W = lambda k: w[f"{p}.{k}.weight"].tolist()
    xn = [b_rms(r, w[f"{p}.pre_attn_norm.weight"].tolist()) for r in x[0].tolist()]
    ks = [b_lin(W("self_attn.k_proj"), r) for r in xn]
    vs = [b_lin(W("self_attn.v_proj"), r) for r in xn]
    for t in range(5):
        q = b_lin(W("self_attn.q_proj"), xn[t])
        o = b_mha(q, ks, vs, [[0.0] * cfg.num_heads] * 5, cfg.num_heads)  # bidirectional, no bias
        y = [a + b for a, b in zip(x[0, t].tolist(), b_lin(W("self_attn.o_proj"), o))]
        yn = b_rms(y, w[f"{p}.pre_ffn_norm.weight"].tolist())
        h = [b_gelu(a) * b for a, b in zip(b_lin(W("ffn.wi_0"), yn), b_lin(W("ffn.wi_1"), yn))]
        exp = [a + b for a, b in zip(y, b_lin(W("ffn.wo"), h))]
        np.testing.assert_allclose(got[0, t], exp, rtol=1e-10, atol=1e-10)


def test_encode_embeds_with_sinusoid_and_final_norm(micro):
    cfg, w, om = micro
    toks = np.array([[3, 7, 1, 0, 17]])
    got = om.encode(toks)
    x = w["token_embedding.weight"][toks] + O.sinusoidal_position_embedding(cfg.max_encoder_length,
                                                                             cfg.d_model)[:5][None]
    x = om.encoder_layer(x, 0)
    np.testing.assert_allclose(got, om.norm(x, "encoder_norm"), rtol=1e-12, atol=1e-12)
    with pytest.raises(IndexError):
        om.encode(np.zeros((1, cfg.max_encoder_length + 1), dtype=np.int64))


# ---- structural invariants ------------------------------------------------------------

def test_depth_step_chain_equals_full_causal_pass(tiny):
    cfg, _, om = tiny
    rng = np.random.default_rng(3)
    embs = rng.standard_normal((2, cfg.rvq_depth, cfg.d_model))
    full = om.depth_forward_full(embs)
    cache = om.empty_depth_cache()
    for l in range(cfg.rvq_depth):
        step = om.depth_step(embs[:, l:l + 1], cache, l)
        np.testing.assert_allclose(step, full[:, l], rtol=1e-9, atol=1e-9)
    # non-causal full pass differs (the mask matters)
    nc = om.depth_forward_full(embs, causal=False)
    assert np.abs(nc[:, 0] - full[:, 0]).max() > 1e-3


def test_temporal_step_chain_equals_full_causal_pass(tiny):
    cfg, _, om = tiny
    rng = np.random.default_rng(4)
    frames = rng.standard_normal((2, 6, cfg.d_model))
    enc = rng.standard_normal((2, 9, cfg.d_model))
    full = om.temporal_forward_full(frames, enc)
    cache = om.empty_temporal_cache()
    for f in range(6):
        out = om.temporal_step(frames[:, f:f + 1], enc, cache, f)
        np.testing.assert_allclose(out[:, 0], full[:, f], rtol=1e-9, atol=1e-9)


def test_kv_rows_are_prefix_projections(tiny):
    cfg, _, om = tiny
    rng = np.random.default_rng(5)
    embs = rng.standard_normal((2, 5, cfg.d_model))
    cache = om.empty_depth_cache()
    for l in range(5):
        om.depth_step(embs[:, l:l + 1], cache, l)
    xn = om.norm(embs, "depth_layers.0.pre_self_attn_norm")
    k = om.linear(xn, "depth_layers.0.self_attn.k_proj")
    v = om.linear(xn, "depth_layers.0.self_attn.v_proj")
    assert cache[0]["k"].shape == (2, cfg.num_heads, 5, cfg.d_kv)
    D = cfg.d_kv
    for h in range(cfg.num_heads):  # head h holds projection elements [h*D, (h+1)*D)
        np.testing.assert_allclose(cache[0]["k"][:, h], k[:, :, h * D:(h + 1) * D], rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(cache[0]["v"][:, h], v[:, :, h * D:(h + 1) * D], rtol=1e-12, atol=1e-12)


def test_ring_mask_equals_concat(tiny):
    cfg, _, om = tiny
    rng = np.random.default_rng(6)
    Lmax, pos = 16, 6
    q = rng.standard_normal((2, cfg.num_heads, 1, 64))
    ring_k = rng.standard_normal((2, cfg.num_heads, Lmax, 64))
    ring_v = rng.standard_normal((2, cfg.num_heads, Lmax, 64))
    bias = om.depth_bias(pos, key_length=Lmax)
    mask = np.where(np.arange(Lmax) <= pos, 0.0, -np.inf)[None, None, None]
    ring = O.sdpa(q, ring_k, ring_v, bias + mask, om.P)
    concat = O.sdpa(q, ring_k[:, :, :pos + 1], ring_v[:, :, :pos + 1], bias[..., :pos + 1], om.P)
    np.testing.assert_allclose(ring, concat, rtol=1e-13, atol=1e-13)


def _teacher(cfg, F, seed):
    rng = np.random.default_rng(seed)
    C = 8  # codebook of the tiny config's levels (2 + 8 * 16 <= vocab)
    lo = 2 + C * np.arange(cfg.rvq_depth)
    return (lo[None, :] + rng.integers(0, C, (F, cfg.rvq_depth))).astype(np.int32), C


def test_depth_cache_reset_and_frame_mean(tiny):
    cfg, w, om = tiny
    F = 3
    teacher, C = _teacher(cfg, F, 7)
    rng = np.random.default_rng(8)
    enc_tokens = rng.integers(0, cfg.vocab_size, (2, cfg.max_encoder_length))
    opts = O.GenerateOptions(num_frames=F, rvq_depth=cfg.rvq_depth, temperature=1.0, top_k=4,
                             guidance_weight=3.0, seed=11, codebook_size=C, codec_offset=2)
    rec = {}
    toks = O.generate_tokens(om, enc_tokens, opts, teacher=teacher, record=rec)
    np.testing.assert_array_equal(toks, teacher)
    E = w["token_embedding.weight"]
    for f in range(F):
        # (iv) a fresh depth chain from this frame's temporal output reproduces the slices
        cache = om.empty_depth_cache()
        x = rec["temporal_out"][f][:, None].astype(np.float64)
        for l in range(cfg.rvq_depth):
            lg = om.depth_step(x, cache, l)
            lo = 2 + C * l
            np.testing.assert_allclose(rec["slices"][f, l], lg[:, lo:lo + C], rtol=1e-6, atol=1e-6)
            x = np.repeat(E[teacher[f, l]][None, None], 2, axis=0)
        # (v) the frame mean is the running sum of the embeddings over rvq_depth
        s = np.zeros(cfg.d_model)
        for l in range(cfg.rvq_depth):
            s = s + E[teacher[f, l]]
        np.testing.assert_allclose(rec["frame_mean"][f], np.repeat((s / cfg.rvq_depth)[None], 2, axis=0),
                                   rtol=1e-6, atol=1e-6)


def test_frame_mean_rounds_each_add_in_bf16(tiny):
    cfg, w, _ = tiny
    om = O.OracleDepthformer({k: v.astype(np.float32) for k, v in w.items()}, cfg, mode="bf16")
    F = 1
    teacher, C = _teacher(cfg, F, 9)
    enc_tokens = np.random.default_rng(10).integers(0, cfg.vocab_size, (2, cfg.max_encoder_length))
    opts = O.GenerateOptions(num_frames=F, rvq_depth=cfg.rvq_depth, codebook_size=C, codec_offset=2)
    rec = {}
    O.generate_tokens(om, enc_tokens, opts, teacher=teacher, record=rec)
    E = om.w["token_embedding.weight"]
    s = E[teacher[0, 0]].astype(np.float32)
    for l in range(1, cfg.rvq_depth):
        s = O.round_bf16(s + E[teacher[0, l]])
    exp = O.round_bf16(s / O.round_bf16(np.float32(cfg.rvq_depth)))
    np.testing.assert_array_equal(rec["frame_mean"][0, 0], exp)
    # a single rounding of the exact mean differs somewhere
    exact = O.round_bf16(E[teacher[0]].astype(np.float64).sum(0) / cfg.rvq_depth)
    assert not np.array_equal(exp, exact)


# ---- the checks catch plausible mistakes (planted in the oracle, CPU only) -------------

def _depth_mismatch(om, w, cfg):
    rng = np.random.default_rng(0)
    embs = rng.standard_normal((1, 4, cfg.d_model))
    cache = om.empty_depth_cache()
    table = w["depth_rel_pos.relative_attention_bias.weight"]
    pk, pv, worst = [], [], 0.0
    for l in range(4):
        got, (k, v), _ = om.decoder_layer(embs[:, l:l + 1], "depth_layers", 0, bias=om.depth_bias(l),
                                          past=None if l == 0 else (cache[0]["k"], cache[0]["v"]))
        cache[0]["k"], cache[0]["v"] = k, v
        exp, bk, bv = b_decoder_step(w, "depth_layers.0", embs[0, l].tolist(), pk, pv,
                                     [table[l - j].tolist() for j in range(l + 1)], cfg.num_heads)
        pk.append(bk)
        pv.append(bv)
        worst = max(worst, float(np.abs(got[0, 0] - np.array(exp)).max()))
    return worst


@pytest.mark.parametrize("mutation", ["sdpa_scale", "bias_offset", "gate_up_swapped", "norm_eps_outside",
                                      "head_split_transposed", "bias_head_reversed"])
def test_planted_mistakes_are_caught(micro, monkeypatch, mutation):
    cfg, w, om = micro
    assert _depth_mismatch(om, w, cfg) < 1e-10
    if mutation == "sdpa_scale":
        real = O.sdpa
        monkeypatch.setattr(O, "sdpa", lambda q, k, v, m, P: real(q / 8.0, k, v, m, P))
    elif mutation == "bias_offset":
        real_b = om.depth_bias
        # query position off by one, same key length
        monkeypatch.setattr(om, "depth_bias", lambda i, **kw: real_b(i + 1, key_length=i + 1))
    elif mutation == "gate_up_swapped":
        def ffn(x, prefix):
            a = om.linear(x, prefix + ".wi_1")
            b = om.linear(x, prefix + ".wi_0")
            return om.linear(om.P.r(O.gelu_approx(a, om.P) * b), prefix + ".wo")
        monkeypatch.setattr(om, "ffn", ffn)
    elif mutation == "norm_eps_outside":
        monkeypatch.setattr(O, "rms_norm",
                            lambda x, g, eps, P: P.r(x / (np.sqrt(np.mean(x * x, -1, keepdims=True)) + 1e-1) * g))
    elif mutation == "head_split_transposed":
        # (B, T, D, H) split with the matching merge: self-consistent, wrong layout
        H, D = cfg.num_heads, cfg.d_kv

        def split(y):
            B, T, _ = y.shape
            return y.reshape(B, T, D, H).transpose(0, 3, 1, 2)

        def merge(o):
            B, _, T, _ = o.shape
            return o.transpose(0, 2, 3, 1).reshape(B, T, H * D)
        monkeypatch.setattr(om, "_heads", split)
        monkeypatch.setattr(om, "_merge_heads", merge)
    elif mutation == "bias_head_reversed":
        real_b = om.depth_bias
        monkeypatch.setattr(om, "depth_bias", lambda i, **kw: real_b(i, **kw)[:, ::-1])
    assert _depth_mismatch(om, w, cfg) > 1e-4
