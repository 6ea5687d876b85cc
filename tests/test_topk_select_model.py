"""The early stop of the top-k threshold selects in the draw kernels and the
restricted-argmax chain of the block draw (draw_block.hpp: the frame kernel and
the per-level samplers), checked as an algorithm on the CPU (numpy models of
the device select and chain; the device code itself is checked draw by draw
against the oracle sampler in the GPU tests).

The select looks for the k-th largest logit (ties counted) over
order-preserving uint32 keys, byte-wise with histograms.  It stops early once
the keys at or above the current prefix (lower digits zero) are exactly the
top-k set, and the draw then keeps v >= float(prefix).  These tests check that the kept set
always equals {v >= k-th largest} (decode.cpp:119-121) on rows with ties,
signed zeros, denormals, all-negative and huge values, so the early stop
cannot change a draw."""

from __future__ import annotations

import numpy as np
import pytest


def _key(v):
    u = v.astype(np.float32).view(np.uint32).astype(np.uint64)
    return np.where(u & 0x80000000, (~u) & 0xFFFFFFFF, u | 0x80000000).astype(np.uint64)


def _key_float(k):
    k = int(k)
    u = (k & 0x7FFFFFFF) if (k & 0x80000000) else ((~k) & 0xFFFFFFFF)
    return np.array([u], dtype=np.uint32).view(np.float32)[0]


def _stop_ok(prefix):
    return prefix != 0x80000000 and np.isfinite(_key_float(prefix))


def byte_select(v, k):
    """Byte-wise select with the early stop (the frame kernel's draw)."""
    key = _key(v)
    prefix, mask, need = 0, 0, k
    for p in range(4):
        sh = 24 - 8 * p
        sel = (key & np.uint64(mask)) == np.uint64(prefix)
        hist = np.bincount(((key[sel] >> np.uint64(sh)) & np.uint64(255)).astype(np.int64), minlength=256)
        above = 0
        for b in range(255, -1, -1):
            if above < need <= above + hist[b]:
                bin_, before, cnt = b, above, int(hist[b])
                break
            above += hist[b]
        prefix |= bin_ << sh
        mask |= 255 << sh
        need -= before
        if p < 3 and cnt == need and _stop_ok(prefix):
            return v >= _key_float(prefix), p
    return v >= _key_float(prefix), 3


def _rows(rng, n):
    for i in range(n):
        kind = i % 5
        if kind == 0:
            v = rng.normal(0, rng.uniform(0.1, 30), 1024)
        elif kind == 1:
            v = np.round(rng.normal(0, 3, 1024), 1)  # many ties
        elif kind == 2:
            v = -np.abs(rng.normal(0, 1e-3, 1024))  # all negative
        elif kind == 3:
            v = rng.choice([0.0, -0.0, 1e-40, -1e-40, 1.0, -1.0, 2.0], 1024)  # signed zeros, denormals
        else:
            v = rng.standard_cauchy(1024) * 1e30
        yield v.astype(np.float32), int(rng.choice([1, 2, 40, 100, 1023]))


def test_early_stop_keeps_the_top_k_set():
    rng = np.random.default_rng(0)
    stops = set()
    for v, k in _rows(rng, 1500):
        exact = v >= np.sort(v)[::-1][k - 1]
        got, p = byte_select(v, k)
        np.testing.assert_array_equal(got, exact)
        stops.add(p)
    assert stops == {0, 1, 2, 3}  # every stopping point was exercised


def test_guarded_thresholds_are_left_to_the_full_select():
    # the k-th largest is a positive denormal and -0 lies below it: a stop at
    # the +0 key (threshold +0.0) would keep -0, which the full select drops
    v = np.array([3.0, 2.0, 1e-45, -0.0, -1.0], dtype=np.float32)
    # the k-th largest is a huge negative value: a stop at the key 0 prefix
    # gives a NaN threshold, which would keep nothing
    w = np.array([1.0, -3.0e38, -3.2e38, -3.3e38], dtype=np.float32)
    # ties at +0 / -0: the float compare keeps both
    z = np.array([3.0, 2.0, 0.0, -0.0, -1.0], dtype=np.float32)
    for x, k in ((v, 3), (w, 4), (w, 2), (z, 3), (z, 4)):
        exact = x >= np.sort(x)[::-1][k - 1]
        np.testing.assert_array_equal(byte_select(x, k)[0], exact)


@pytest.mark.parametrize("k", [40])
def test_normal_logits_stop_after_two_or_three_bytes(k):
    rng = np.random.default_rng(1)
    passes = [byte_select((rng.normal(0, 2.0, 1024) / 1.1).astype(np.float32), k)[1] for _ in range(300)]
    assert max(passes) <= 2 or np.mean(np.array(passes) <= 2) > 0.95


def _masked_argmax(v, g, k):
    """The reference's draw: argmax of v + g over {v >= k-th largest v}, the
    smallest index among equal maxima (decode.cpp:119-125, mx::argmax)."""
    keep = v >= np.sort(v)[::-1][k - 1]
    w = np.where(keep, v + g, -np.inf).astype(np.float32)
    return int(np.argmax(w))


def chain_draw(v, g, k, steps):
    """The frame kernel's draw (sample_block): the unmasked winner, then up to
    `steps` winners restricted to {v > v_prev}, each accepted once fewer than k
    values exceed it; else the exact threshold (the radix select's set).
    Returns (index, the number of restricted steps taken, fell back)."""
    w = (v + g).astype(np.float32)
    a = int(np.argmax(w))
    taken = 0
    while (v > v[a]).sum() >= k:
        if taken == steps:
            return _masked_argmax(v, g, k), taken, True
        w = np.where(v > v[a], (v + g).astype(np.float32), -np.inf)
        a = int(np.argmax(w))
        taken += 1
    return a, taken, False


def test_chain_steps_give_the_masked_draw():
    """Every draw of the restricted-argmax chain equals the reference's masked
    draw, on rows with ties in v and in v + g, signed zeros, denormals and
    huge values, for chain lengths 0..3 (0: the fast path, then the select)."""
    rng = np.random.default_rng(2)
    taken_seen = set()
    for i, (v, k) in enumerate(_rows(rng, 1500)):
        if i % 3 == 0:
            g = rng.choice([0.0, 0.5, 1.0], v.size).astype(np.float32)  # ties in v + g
        else:
            g = (-np.log(-np.log(rng.random(v.size)))).astype(np.float32)
        want = _masked_argmax(v, g, k)
        for steps in (0, 1, 3):
            got, taken, _ = chain_draw(v, g, k, steps)
            assert got == want, (i, k, steps)
            taken_seen.add(taken)
    assert {0, 1, 2, 3} <= taken_seen  # every chain length was exercised


def test_chain_steps_spare_most_selects_on_flat_logits():
    """Flat guided logits (the random-weight benchmark's): the chain of 3
    settles most draws that miss the fast path without the radix select."""
    rng = np.random.default_rng(3)
    fell = [chain_draw((rng.normal(0, 1.0, 1024) / 1.1).astype(np.float32),
                       (-np.log(-np.log(rng.random(1024)))).astype(np.float32), 40, 3)[2] for _ in range(400)]
    assert np.mean(fell) < 0.2
