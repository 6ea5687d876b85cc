"""The draw checker used by the GPU tests accepts exactly the oracle's draw and
ulp-level ties of its scaled + noise, and rejects the mistakes a wrong top-k
select or index would make (planted here, on the CPU)."""

from __future__ import annotations

import numpy as np

from draw_check import assert_argmax_flips_are_near_ties, check_draw
from oracle import depthformer_oracle as O

KW = dict(temperature=1.1, top_k=40, seed=5, frame=3, level=7)


def _guided(seed=0, n=1024):
    rng = np.random.default_rng(seed)
    return O.cfg_combine((rng.standard_normal((2, n)) * 3).astype(np.float32), 5.0)


def test_oracle_draw_passes():
    g = _guided()
    exp = O.sample_level(g, **KW)
    assert check_draw(O, g, exp, **KW) == (exp, None)


def test_runner_up_outside_a_tie_fails():
    g = _guided()
    exp = O.sample_level(g, **KW)
    scaled = O.top_k_logits((g / np.float32(1.1)).astype(np.float32), 40)
    v = scaled + O.gumbel_noise(5, 3, 7, g.size)
    v[exp] = -np.inf
    second = int(np.argmax(v))  # best other candidate of the top-k set
    _, msg = check_draw(O, g, second, **KW)
    assert msg is not None and "gap" in msg


def test_draw_outside_top_k_fails():
    g = _guided(1)
    scaled = (g / np.float32(1.1)).astype(np.float32)
    outside = int(np.argsort(scaled)[0])  # the smallest logit is never in the top 40
    _, msg = check_draw(O, g, outside, **KW)
    assert msg is not None and "outside the top-40" in msg


def test_exact_tie_passes():
    # make a top-k candidate's scaled + noise equal the winner's to the last bit
    g = _guided(2).astype(np.float32)
    exp = O.sample_level(g, **KW)
    noise = O.gumbel_noise(5, 3, 7, g.size)
    scaled = (g / np.float32(1.1)).astype(np.float32)
    order = np.argsort(scaled)[::-1]
    other = int(order[0] if order[0] != exp else order[1])
    target = np.float32(scaled[exp] + noise[exp] - noise[other])  # wanted scaled[other]
    # search the float32 neighbourhood of target * 1.1 for a logit that scales onto it
    cand = np.float32(target * np.float32(1.1))
    for _ in range(64):
        if np.float32(cand / np.float32(1.1)) >= target:
            break
        cand = np.nextafter(cand, np.float32(np.inf))
    g2 = g.copy()
    g2[other] = cand
    if O.sample_level(g2, **KW) == other:  # the nudge made it the outright winner
        return
    _, msg = check_draw(O, g2, other, **KW)
    assert msg is None, msg


def test_argmax_at_temperature_zero_is_exact():
    g = _guided(3)
    exp = int(np.argmax(g))
    kw = dict(KW, temperature=0.0)
    assert check_draw(O, g, exp, **kw)[1] is None
    assert check_draw(O, g, (exp + 1) % g.size, **kw)[1] is not None


def test_argmax_flip_rule():
    from draw_check import guided
    rng = np.random.default_rng(4)
    ref = rng.standard_normal((2, 3, 2, 1024)).astype(np.float64)
    noisy = ref + 1e-3 * rng.standard_normal(ref.shape)
    assert_argmax_flips_are_near_ties(noisy, ref)
    # a flip from noise on every candidate whose scale reaches the margin passes
    g0 = guided(ref)[0, 0]
    top = np.sort(g0)
    margin = top[-1] - top[-2]
    spread = ref.copy()
    spread[0, 0, 0] += (margin / 6) * rng.standard_normal(1024) / 6  # rms of the guided error ~ margin / 6
    w, r = g0.argmax(), np.argsort(g0)[-2]
    spread[0, 0, 0, w] -= margin / 12
    spread[0, 0, 0, r] += margin / 12
    if guided(spread)[0, 0].argmax() != w:
        assert_argmax_flips_are_near_ties(spread, ref)
    # the same flip from an error confined to the winner fails
    bad = ref.copy()
    bad[0, 0, 0, w] -= (margin + 0.05) / 6  # guided winner drops below the runner-up
    assert guided(bad)[0, 0].argmax() != w
    try:
        assert_argmax_flips_are_near_ties(bad, ref)
    except AssertionError:
        return
    raise AssertionError("a flip from a one-candidate error passed")
