"""Pins of the oracle's math against closed forms and independent library routines."""

import math

import numpy as np
import pytest
import torch

from oracle import depthformer_oracle as O


# ---- relative position buckets (modules.cpp:139-174) ------------------------------

def _bucket_float64(n, num_buckets, max_distance):
    max_exact = num_buckets // 2
    if n < max_exact:
        return n
    v = max_exact + math.log(n / max_exact) / math.log(max_distance / max_exact) * (num_buckets - max_exact)
    return min(int(v), num_buckets - 1)


@pytest.mark.parametrize("nb,md", [(16, 16), (128, 128), (32, 128)])
def test_bucket_vs_float64_bruteforce(nb, md):
    n = np.arange(0, 400)
    got = O.relative_position_bucket(-n, False, nb, md)  # rel = k - q = -n
    exp = [_bucket_float64(int(v), nb, md) for v in n]
    assert got.tolist() == exp


def test_bucket_closed_form_identity():
    # depth 16/16 over 0..15 and temporal 128/128 over 0..49: bucket == distance
    assert O.relative_position_bucket(-np.arange(16), False, 16, 16).tolist() == list(range(16))
    assert O.relative_position_bucket(-np.arange(50), False, 128, 128).tolist() == list(range(50))
    # future keys (k > q) map to bucket 0 in the unidirectional case
    assert O.relative_position_bucket(np.arange(1, 9), False, 16, 16).tolist() == [0] * 8


def test_rel_pos_bias_gather():
    rng = np.random.default_rng(0)
    table = rng.standard_normal((16, 3)).astype(np.float32)
    b = O.rel_pos_bias(table, 1, 6, 5, 16, 16)
    assert b.shape == (1, 3, 1, 6)
    for h in range(3):
        for k in range(6):
            assert b[0, h, 0, k] == table[5 - k, h]


# ---- sinusoidal PE (model.cpp:54-80) ------------------------------------------------

def test_sinusoid_closed_form():
    pe = O.sinusoidal_position_embedding(1006, 1024)
    half = 512
    pos = np.arange(1006)[:, None].astype(np.float64)
    i = np.arange(half)[None, :].astype(np.float64)
    ang = pos * np.exp(-i * math.log(1e4) / (half - 1))
    np.testing.assert_allclose(pe[:, :half], np.sin(ang), atol=2e-4)
    np.testing.assert_allclose(pe[:, half:], np.cos(ang), atol=2e-4)
    assert pe[0, :half].tolist() == [0.0] * half and pe[0, half:].tolist() == [1.0] * half


# ---- elementwise -----------------------------------------------------------------

def test_gelu_approx_vs_exact_gelu():
    x = np.linspace(-6, 6, 2001)
    got = O.gelu_approx(x, O.Precision("fp64"))
    exact = torch.nn.functional.gelu(torch.tensor(x), approximate="none").numpy()
    assert np.max(np.abs(got - exact)) < 1e-3
    tanh_ref = torch.nn.functional.gelu(torch.tensor(x), approximate="tanh").numpy()
    # the constants are float32 literals (nn_ops.h:76-79): ~1e-7 relative
    np.testing.assert_allclose(got, tanh_ref, rtol=1e-6, atol=1e-12)


def test_rms_norm_vs_torch():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 5, 64)) * 3
    w = 1 + 0.1 * rng.standard_normal(64)
    got = O.rms_norm(x, w, 1e-6, O.Precision("fp64"))
    exp = torch.nn.functional.rms_norm(torch.tensor(x), (64,), torch.tensor(w), eps=1e-6).numpy()
    np.testing.assert_allclose(got, exp, rtol=1e-12, atol=1e-12)


def test_sdpa_vs_torch():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((2, 4, 3, 16))
    k = rng.standard_normal((2, 4, 7, 16))
    v = rng.standard_normal((2, 4, 7, 16))
    bias = rng.standard_normal((1, 4, 3, 7))
    got = O.sdpa(q, k, v, bias, O.Precision("fp64"))
    exp = torch.nn.functional.scaled_dot_product_attention(
        torch.tensor(q), torch.tensor(k), torch.tensor(v), attn_mask=torch.tensor(bias), scale=1.0).numpy()
    np.testing.assert_allclose(got, exp, rtol=1e-10, atol=1e-12)


def test_round_bf16_vs_torch():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 1e-40, 65504.0, 3.3895314e38, np.inf, -np.inf], dtype=np.float32)])
    exp = torch.tensor(x).to(torch.bfloat16).to(torch.float32).numpy()
    got = O.round_bf16(x)
    np.testing.assert_array_equal(got, exp)


def test_round_fp16_closed_forms():
    """binary16 rounding of the fp16 mode: every half value is fixed, midpoints
    between neighbours go to the even one, the overflow and underflow edges sit
    where IEEE 754 puts them, and torch's conversion agrees on random data."""
    halves = np.arange(0x10000, dtype=np.uint32).astype(np.uint16).view(np.float16)
    fin = halves[np.isfinite(halves)].astype(np.float32)
    np.testing.assert_array_equal(O.round_fp16(fin), fin)
    pos = np.sort(np.unique(fin[fin >= 0]))
    lo, hi = pos[:-1].astype(np.float64), pos[1:].astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)  # exact in float32
    even = np.where((pos[:-1].astype(np.float16).view(np.uint16) & 1) == 0, lo, hi).astype(np.float32)
    np.testing.assert_array_equal(O.round_fp16(mid), even)
    np.testing.assert_array_equal(O.round_fp16(-mid), -even)
    edge = np.array([65519.996, 65520.0, 2.0 ** -25, np.nextafter(np.float32(2.0 ** -25), 1), 2.0 ** -24 * 1.5],
                    dtype=np.float32)
    np.testing.assert_array_equal(O.round_fp16(edge), np.array([65504.0, np.inf, 0.0, 2.0 ** -24, 2.0 ** -23],
                                                               dtype=np.float32))
    rng = np.random.default_rng(5)
    x = rng.standard_normal(100000).astype(np.float32) * 100
    np.testing.assert_array_equal(O.round_fp16(x), torch.tensor(x).to(torch.float16).to(torch.float32).numpy())
    assert O.Precision("fp16").r(np.float32(1.0 + 2.0 ** -12)) == np.float32(1.0)  # ties to even at 1 + 2^-11 / 2


# ---- sampling pieces (decode.cpp:71-148) ----------------------------------------------

def test_cfg_combine_properties():
    rng = np.random.default_rng(4)
    l = rng.standard_normal((2, 50)).astype(np.float32)
    np.testing.assert_array_equal(O.cfg_combine(l, 0.0), l[0])
    same = np.stack([l[0], l[0]])
    np.testing.assert_allclose(O.cfg_combine(same, 5.0), l[0], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(O.cfg_combine(l, 5.0), 6.0 * l[0] - 5.0 * l[1], rtol=1e-5, atol=1e-5)


def test_top_k_ties_kept():
    x = np.array([5, 5, 5, 4, 3], dtype=np.float32)
    out = O.top_k_logits(x, 2)
    assert np.isfinite(out).tolist() == [True, True, True, False, False]
    out = O.top_k_logits(np.array([1, 9, 3, 7, 5], dtype=np.float32), 3)
    assert np.isfinite(out).tolist() == [False, True, False, True, True]


def test_philox_known_answers():
    # Random123 known-answer vectors for philox4x32_10.
    kat = [
        ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
        ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
        ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
         (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
    ]
    for ctr, key, exp in kat:
        got = O.philox4x32_10([np.array([c], dtype=np.uint64) for c in ctr], key)
        assert tuple(int(g[0]) for g in got) == exp


def test_gumbel_range_and_moments():
    g = O.gumbel_noise(7, 3, 2, 200000)
    assert np.all(np.isfinite(g))
    assert abs(g.mean() - 0.5772156649) < 0.01          # Euler-Mascheroni
    assert abs(g.var() - math.pi ** 2 / 6) < 0.03


def test_sampling_distribution_chi_square():
    from scipy import stats
    rng = np.random.default_rng(5)
    C, k, T = 16, 5, 1.1
    guided = rng.standard_normal(C).astype(np.float32) * 2
    scaled = (guided / np.float32(T)).astype(np.float32)
    kept = O.top_k_logits(scaled, k)
    p = np.exp(kept - kept.max())
    p /= p.sum()
    n = 20000
    counts = np.zeros(C)
    for s in range(n):
        counts[O.sample_level(guided, temperature=T, top_k=k, seed=s, frame=0, level=0)] += 1
    assert counts[p == 0].sum() == 0
    nz = p > 0
    chi2, pval = stats.chisquare(counts[nz], n * p[nz])
    assert pval > 1e-3, (chi2, pval)


def test_argmax_at_zero_temperature():
    g = np.array([0.1, 3.0, 3.0, -1.0], dtype=np.float32)
    assert O.sample_level(g, temperature=0.0, top_k=40, seed=0, frame=0, level=0) == 1
