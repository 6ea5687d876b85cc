"""Device draws against the oracle sampler, with every disagreement examined.

The device and the oracle compute the same guided, temperature-scaled logits
bit for bit (CFG ``(1+w)*l0 - w*l1`` without a fused multiply-add, then one
IEEE division).  Only the Gumbel noise differs, by the last bits of two float32
``log`` implementations (the device's ``logf`` and numpy's).  So a device draw
may differ from the oracle's only where two candidates of the top-k set are
within a few ulps of each other in ``scaled + noise``.  ``assert_draws`` fails on
any other disagreement: a draw outside the oracle's top-k set, or one whose
value in the oracle's ``scaled + noise`` is more than ``TIE_ULPS`` ulps below the
oracle's winner.  A wrong top-k threshold, select or index fails it.
"""

from __future__ import annotations

import numpy as np

# ulps of the compared magnitude: -log(-log(u)) with each log within 2 ulps
# moves g by a few ulps of max(|g|, 1); both candidates' noise can move.
TIE_ULPS = 16


def _noisy(O, guided, temperature, top_k, seed, frame, level):
    g = np.asarray(guided, dtype=np.float32)
    scaled = (g / np.float32(temperature)).astype(np.float32)
    if top_k > 0:
        scaled = O.top_k_logits(scaled, min(top_k, scaled.size))
    noise = O.gumbel_noise(seed, frame, level, scaled.size)
    return scaled, noise, (scaled + noise).astype(np.float32)


def check_draw(O, guided, got_index, *, temperature, top_k, seed, frame, level):
    """Returns ``(oracle_index, message)``: message is None when ``got_index`` is
    the oracle's draw or an ulp-level tie with it, else it names the disagreement.
    At temperature 0 (argmax, first maximum) only the exact index passes."""
    exp = O.sample_level(guided, temperature=temperature, top_k=top_k, seed=seed, frame=frame, level=level)
    if got_index == exp:
        return exp, None
    if not 0 <= got_index < len(guided):
        return exp, f"index {got_index} outside the slice"
    if temperature == 0.0:
        g = np.asarray(guided, dtype=np.float32)
        return exp, f"argmax {got_index} ({g[got_index]!r}) vs {exp} ({g[exp]!r})"
    scaled, noise, v = _noisy(O, guided, temperature, top_k, seed, frame, level)
    if not np.isfinite(scaled[got_index]):
        return exp, f"draw {got_index} is outside the top-{top_k} set (oracle {exp})"
    mag = np.float32(max(abs(float(v[exp])), abs(float(noise[exp])), abs(float(noise[got_index])), 1.0))
    gap = float(v[exp]) - float(v[got_index])
    tol = TIE_ULPS * float(np.spacing(mag))
    if gap > tol:
        return exp, (f"draw {got_index} (scaled+noise {v[got_index]!r}) vs oracle {exp} ({v[exp]!r}): "
                     f"gap {gap:.3e} > {tol:.3e}")
    return exp, None


def assert_draws(O, drawn, guided, *, temperature, top_k, seed, offset, codebook, max_ties=None):
    """``drawn[f, l]`` (absolute ids) against the oracle's draws from ``guided[f, l]``
    (the CFG-combined slice of frame f, level l).  Every mismatch must be a tie
    (``check_draw``); ``max_ties`` bounds how many ties may occur.  Returns the
    number of ties."""
    drawn = np.asarray(drawn)
    F, L = drawn.shape
    ties, bad = 0, []
    for f in range(F):
        for l in range(L):
            idx = int(drawn[f, l]) - offset - codebook * l
            exp, msg = check_draw(O, guided[f, l], idx, temperature=temperature, top_k=top_k, seed=seed, frame=f,
                                  level=l)
            if msg is not None:
                bad.append((f, l, msg))
            elif idx != exp:
                ties += 1
    assert not bad, bad[:8]
    if max_ties is not None:
        assert ties <= max_ties, (ties, max_ties)
    return ties


def guided(slices, w=5.0):
    """CFG combine of (..., 2, C) level slices in float64: (1+w) l0 - w l1."""
    s = np.asarray(slices, dtype=np.float64)
    return (1 + w) * s[..., 0, :] - w * s[..., 1, :]


FLIP_SIGMAS = 8.0


def assert_argmax_flips_are_near_ties(got_slices, ref_slices, w=5.0):
    """Teacher-forced CFG argmax of ``got`` against ``ref`` ((F, L, 2, C) slices).
    Two 16-bit evaluations differ by rounding noise spread over every candidate,
    which guidance weight w amplifies; an argmax may flip only where the
    reference's top-1 / top-2 margin is within ``FLIP_SIGMAS`` times the RMS of
    that draw's guided-logit error.  (Bounding the margin by the draw's largest
    error instead would hold for every flip by construction: a flip needs the
    two candidates' errors to add up to at least the margin.)  An error confined
    to a few candidates -- a wrong index, a dropped term on one row -- hardly
    moves the RMS over C candidates, so a flip it causes fails here.  Returns the
    agreement fraction."""
    gl, ol = guided(got_slices, w), guided(ref_slices, w)
    ga, oa = gl.argmax(-1), ol.argmax(-1)
    top2 = np.sort(ol, -1)
    margin = top2[..., -1] - top2[..., -2]
    rms = np.sqrt(np.mean((gl - ol) ** 2, -1))
    flips = ga != oa
    ok = margin[flips] <= FLIP_SIGMAS * rms[flips]
    assert ok.all(), [(tuple(i), float(m), float(r)) for i, m, r in
                      zip(np.argwhere(flips)[~ok], margin[flips][~ok], rms[flips][~ok])]
    return float((~flips).mean())
