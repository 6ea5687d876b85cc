"""bf16 parity of whole chunks against exact arithmetic.

Two bf16 evaluations of the model that round at the same op boundaries but
accumulate in different orders (the HIP kernels, MLX, the oracle's bf16
restatement) differ from each other by independent rounding noise of the same
size, so a bf16 implementation is compared with the fp32 oracle (exact up to
fp32 rounding), and its error is compared with the error of a reference bf16
evaluation (the oracle's bf16 mode) against the same fp32 oracle:

  * per (frame, level) slice of 1024 codes: rel(got, fp32) <= TOL (2e-2, the
    bf16 logit tolerance);
  * over the chunk: rms over slices of rel(got, fp32) <= (1 + DELTA) x the
    same for the bf16 oracle -- the implementation's rounding error is no
    larger than a bf16 evaluation's (a systematic error, such as a dropped or
    misplaced rounding in one op, adds to every slice and fails this);
  * CFG argmax (guidance weight w) of got against the fp32 oracle agrees at
    least as often as the bf16 oracle's does, less SLACK, and every flip is a
    near-tie (draw_check.assert_argmax_flips_are_near_ties against fp32).
"""

from __future__ import annotations

import numpy as np
from draw_check import assert_argmax_flips_are_near_ties, guided

TOL = 2e-2
DELTA = 0.25
SLACK = 0.05


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def slice_errors(got, ref):
    """(F, L) norm-wise relative errors of (F, L, 2, C) slices."""
    F, L = got.shape[:2]
    return np.array([[rel(got[f, l], ref[f, l]) for l in range(L)] for f in range(F)])


def argmax_agreement(a, b, w=5.0):
    return float((guided(a, w).argmax(-1) == guided(b, w).argmax(-1)).mean())


def assert_bf16_chunk(got, o16, o32, w=5.0, tol=TOL, delta=DELTA, slack=SLACK):
    """got / o16 / o32: (F, L, 2, C) level slices of the implementation, the
    bf16 oracle and the fp32 oracle on the same fed tokens.  Returns the
    figures (for the log)."""
    e_got = slice_errors(got, o32)
    e_ref = slice_errors(o16, o32)
    rms_got = float(np.sqrt(np.mean(e_got ** 2)))
    rms_ref = float(np.sqrt(np.mean(e_ref ** 2)))
    a_got = argmax_agreement(got, o32, w)
    a_ref = argmax_agreement(o16, o32, w)
    figs = dict(max_slice=float(e_got.max()), rms_slice=rms_got, ref_max_slice=float(e_ref.max()),
                ref_rms_slice=rms_ref, ratio=rms_got / rms_ref, argmax=a_got, ref_argmax=a_ref,
                vs_bf16_max_slice=float(slice_errors(got, o16).max()))
    assert e_got.max() <= tol, (figs, np.unravel_index(e_got.argmax(), e_got.shape))
    assert rms_got <= (1.0 + delta) * rms_ref, figs
    assert a_got >= a_ref - slack, figs
    assert_argmax_flips_are_near_ties(got, o32, w)
    return figs
