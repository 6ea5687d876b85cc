"""The XCD-grouped tile order of the encoder GEMM (`grouped_tile` in
encoder_kernels.hip), checked as index arithmetic on the CPU: block L of a
1-D grid must map to a distinct in-range tile for every L < tm * tn, so that
every output tile is computed exactly once, whatever the shape and group
height.  The device kernels themselves are checked bit for bit against the
2-D-grid tiling in the GPU tests (every tile shape accumulates an output over
k in the same order).

The model restates the kernel's integer formulas: blocks are dealt to the 8
XCDs in turn (XCD L % 8), XCD x takes the contiguous id range starting at
x * (T / 8) + min(x, T % 8), and ids run down GM row tiles before the next
column tile (the last group of rows may be shorter)."""

from __future__ import annotations

import numpy as np
import pytest


def grouped_tile(L, tm, tn, gm):
    tiles = tm * tn
    x, q, rem = L & 7, tiles >> 3, tiles & 7
    pid = x * q + min(x, rem) + (L >> 3)
    g = pid // (gm * tn)
    first = g * gm
    gsz = min(tm - first, gm)
    w = pid - g * gm * tn
    return first + w % gsz, w // gsz


# (rows M, outputs N, tile BM x BN, group) of every launch the dispatcher
# makes with a grouped order at 1, 8 and 32 streams (2 x 1006 rows each), plus
# small and odd shapes
SHAPES = [(2012 * b, n, bm, bn, gm) for b in (1, 8, 32)
          for (n, bm, bn, gm) in ((1024, 64, 128, 4), (40960, 256, 256, 4), (1024, 192, 128, 2),
                                  (5632, 192, 128, 4))]
SHAPES += [(1, 128, 64, 128, 4), (65, 256, 64, 128, 4), (1000, 384, 192, 128, 2), (7 * 256 + 3, 2560, 256, 256, 4),
           (120, 384, 64, 128, 4), (300, 1152, 64, 128, 8), (5000, 128, 192, 128, 16)]


@pytest.mark.parametrize("M,N,BM,BN,GM", SHAPES)
def test_grouped_tile_order_is_a_bijection(M, N, BM, BN, GM):
    tm, tn = (M + BM - 1) // BM, N // BN
    seen = np.zeros((tm, tn), dtype=np.int64)
    for L in range(tm * tn):
        mt, nt = grouped_tile(L, tm, tn, GM)
        assert 0 <= mt < tm and 0 <= nt < tn, (L, mt, nt)
        seen[mt, nt] += 1
    assert (seen == 1).all()


def test_grouped_tile_order_keeps_an_xcd_on_few_tiles():
    """The blocks one XCD runs together (its first 32 ids, one per CU of the
    XCD) touch at most GM row tiles and ceil(32 / GM) + 1 column tiles, far
    fewer than the row-major order's 32 column tiles of one row."""
    tm, tn, gm = 252, 160, 4  # the cross K/V projection at 32 streams, 256 x 256 tiles
    tiles = tm * tn
    for x in range(8):
        blocks = [x + 8 * i for i in range(32) if x + 8 * i < tiles]
        rows, cols = set(), set()
        for L in blocks:
            mt, nt = grouped_tile(L, tm, tn, gm)
            rows.add(mt)
            cols.add(nt)
        assert len(rows) <= gm and len(cols) <= 32 // gm + 1, (x, len(rows), len(cols))
