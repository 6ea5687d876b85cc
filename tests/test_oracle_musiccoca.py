"""Pins of the MusicCoCa text-path oracle: torch (float64) for LayerNorm and
attention, math.erf for GELU, closed forms for softplus and the logit cap,
brute-force loops for the attention core and the RVQ argmin, and the RVQ
round trip."""

from __future__ import annotations

import math

import numpy as np
import pytest

import synth_bundle
from oracle import musiccoca_oracle as M


def test_softplus_gelu_closed_forms():
    x = np.array([-30.0, -2.0, 0.0, 0.5, 40.0])
    np.testing.assert_allclose(M.softplus(x), [math.log1p(math.exp(v)) for v in x], rtol=1e-12)
    np.testing.assert_allclose(M.gelu(x), [v * 0.5 * (1 + math.erf(v / math.sqrt(2))) for v in x], rtol=1e-12)


def test_layer_norm_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    x, w, b = rng.standard_normal((5, 16)), rng.standard_normal(16), rng.standard_normal(16)
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x), (16,), torch.from_numpy(w), torch.from_numpy(b),
                                         eps=1e-5).numpy()
    np.testing.assert_allclose(M.layer_norm(x, w, b), ref, rtol=1e-12, atol=1e-12)


def _mha_weights(rng, d, H, D):
    p = {}
    for n, (o, i) in {"q": (H * D, d), "k": (H * D, d), "v": (H * D, d), "o": (d, H * D)}.items():
        p[f"a.{n}_proj.weight"] = rng.standard_normal((o, i)) / math.sqrt(i)
        p[f"a.{n}_proj.bias"] = 0.1 * rng.standard_normal(o)
    p["a._per_dim_scale"] = rng.standard_normal(D)
    return p


def test_mha_brute_force_with_cap_mask_and_scale():
    rng = np.random.default_rng(2)
    d, H, D, S = 8, 2, 4, 5
    p = _mha_weights(rng, d, H, D)
    x = rng.standard_normal((S, d)) * 3.0
    mask = np.array([0, 0, -1e9, 0, -1e9])
    got = M.mha(x, x, x, p, "a", H, D, cap=2.0, mask=mask, per_dim_scale=True)
    q = x @ p["a.q_proj.weight"].T + p["a.q_proj.bias"]
    k = x @ p["a.k_proj.weight"].T + p["a.k_proj.bias"]
    v = x @ p["a.v_proj.weight"].T + p["a.v_proj.bias"]
    sc = np.log1p(np.exp(p["a._per_dim_scale"])) / math.log(2)
    out = np.zeros((S, H * D))
    for h in range(H):
        for i in range(S):
            logits = []
            for j in range(S):
                s = sum(q[i, h * D + t] * sc[t] * k[j, h * D + t] for t in range(D)) / math.sqrt(D)
                logits.append(2.0 * math.tanh(s / 2.0) + mask[j])
            m = max(logits)
            e = [math.exp(l - m) for l in logits]
            for j in range(S):
                out[i, h * D:(h + 1) * D] += e[j] / sum(e) * v[j, h * D:(h + 1) * D]
    ref = out @ p["a.o_proj.weight"].T + p["a.o_proj.bias"]
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)


def test_attention_core_matches_torch_sdpa():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    d, H, D, S = 16, 4, 4, 7
    p = _mha_weights(rng, d, H, D)
    for n in "qkvo":  # identity projections isolate the attention core
        p[f"a.{n}_proj.weight"] = np.eye(d)
        p[f"a.{n}_proj.bias"] = np.zeros(d)
    x = rng.standard_normal((S, d))
    got = M.mha(x, x, x, p, "a", H, D)
    t = torch.from_numpy(x).reshape(S, H, D).transpose(0, 1)
    ref = torch.nn.functional.scaled_dot_product_attention(t, t, t).transpose(0, 1).reshape(S, d).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_text_ids_layout():
    ids, pad = M.text_ids([5, 6, 7], max_len=6)
    np.testing.assert_array_equal(ids, [1, 5, 6, 7, 0, 0])
    np.testing.assert_array_equal(pad, [0, 0, 0, 0, 1, 1])
    ids, pad = M.text_ids(list(range(10, 20)), max_len=4)  # trimmed to leave room for BOS
    np.testing.assert_array_equal(ids, [1, 10, 11, 12])
    assert not pad.any()


def test_rvq_quantization_brute_force_and_round_trip():
    rng = np.random.default_rng(4)
    cb = rng.standard_normal((3, 16, 8)).astype(np.float32)
    v = rng.standard_normal((4, 8)).astype(np.float32)
    tok, res = M.rvq_quantization(v, cb)
    r = v.astype(np.float64)
    for k in range(3):
        for n in range(4):
            dist = [float(np.sum((r[n] - cb[k, c]) ** 2)) for c in range(16)]
            assert tok[n, k] == int(np.argmin(dist))
        r = r - cb[k][tok[:, k]]
    np.testing.assert_allclose(res, r, rtol=1e-5, atol=1e-6)
    # round trip: levels at scales 100, 10, 1 -> each level's nearest code is the planted one
    base = np.eye(8, dtype=np.float32)
    cbs = np.stack([s * np.concatenate([base, -base]) for s in (100.0, 10.0, 1.0)])
    want = np.array([[3, 9, 12], [0, 15, 1]])
    vec = sum(cbs[k][want[:, k]] for k in range(3))
    t2, r2 = M.rvq_quantization(vec, cbs)
    np.testing.assert_array_equal(t2, want)
    assert np.abs(r2).max() == 0


def test_tiny_encoder_runs_and_layout():
    cfg = M.CocaConfig.tiny()
    w = synth_bundle.make_coca_weights(cfg)
    for name, shp in synth_bundle.coca_layout(cfg):
        assert w[name].shape == shp
    o = M.OracleCoca(w, cfg, "fp64")
    ids, pad = M.text_ids([5, 17, 99, 3], cfg.max_text_len)
    e = o.embed_text(ids, pad)
    assert e.shape == (cfg.d_model,) and np.isfinite(e).all()
    st = o.style_tokens_lm(ids, pad, 6, cfg.codebook_size, 100)
    assert st.shape == (6,) and ((st - 100 - cfg.codebook_size * np.arange(6)) < cfg.codebook_size).all()
