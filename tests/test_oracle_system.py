"""Oracle integer plumbing vs the upstream known-answer tests (restated).

Sources: vendor/magenta-realtime/magenta_rt/system_test.py:29-48,
depthformer/decode_test.py:38-50, utils_test.py:99-149; C++ constants
system.h:44-83, system.cpp:62-95, 135-157, 320-333.
"""

import numpy as np
import pytest

from oracle import system_oracle as so


def test_vocab_layout_known_answers():
    c = so.SystemConfig()
    assert c.vocab_mask_token() == 1            # PAD = 0, MASK = 1
    assert c.vocab_codec_offset() == 2
    assert c.vocab_codec_size() == 16384
    assert c.vocab_codec_offset() + c.vocab_codec_size() == 16386
    assert c.vocab_style_offset() == 17410
    assert c.vocab_style_offset() + 6 * 1024 == 23554  # style size 6144
    assert c.chunk_length_frames() == 50
    assert c.context_length_frames() == 250
    assert c.encoder_length() == 1006


def test_level_ranges_match_upstream_acoustic_mask():
    # decode_test.py:38-50: position i >= 250 keeps [2 + l*1024, 2 + (l+1)*1024), l = (i-250) % 4
    c = so.SystemConfig()
    masks = so.build_vocab_masks(c)
    for i in range(250, 2250, 37):
        lvl = (i - 250) % 4
        exp = np.zeros(c.llm_vocab_size, dtype=bool)
        exp[2 + lvl * 1024: 2 + (lvl + 1) * 1024] = True
        np.testing.assert_array_equal(masks[lvl], exp)
    assert masks.sum(axis=1).tolist() == [1024] * 16
    # levels are disjoint and tile [2, 16386)
    assert masks.any(axis=0).sum() == 16384 and not masks.any(axis=0)[:2].any()


RVQ_CASES = [
    ([0, 0, 0, 0], 1024, 0, [0, 1024, 2048, 3072]),
    ([0, 0, 0, 0], 2, 4, [4, 6, 8, 10]),
    ([0, 1, 2, 3], 1024, 0, [0, 1025, 2050, 3075]),
    ([6, 4, 2, 0], 8, 0, [6, 12, 18, 24]),
    ([[0, 0, 0, 0], [0, 1, 2, 3]], 1024, 0, [[0, 1024, 2048, 3072], [0, 1025, 2050, 3075]]),
    ([3], 4, 0, [3]),
    ([], 1024, 0, []),
]


@pytest.mark.parametrize("rvq,cb,off,llm", RVQ_CASES)
def test_rvq_llm_known_answers(rvq, cb, off, llm):
    rvq = np.array(rvq, dtype=np.int32)
    llm = np.array(llm, dtype=np.int32)
    assert so.rvq_to_llm(rvq, cb, off).tolist() == llm.tolist()
    assert so.llm_to_rvq(llm, cb, off).tolist() == rvq.tolist()
    if not np.array_equal(rvq, llm):
        with pytest.raises(IndexError):
            so.rvq_to_llm(llm, cb)
        with pytest.raises(IndexError):
            so.llm_to_rvq(rvq, cb)


def test_rvq_llm_failure_cases():
    with pytest.raises(ValueError):
        so.rvq_to_llm(np.array(0, dtype=np.int32), 1024)
    with pytest.raises(IndexError):
        so.rvq_to_llm(np.array([2]), 2)
    with pytest.raises(IndexError):
        so.rvq_to_llm(np.array([-1]), 2)
    with pytest.raises(ValueError):
        so.llm_to_rvq(np.array(0, dtype=np.int32), 1024)
    for case in [[3, 0], [3], [0, 0], [-1]]:
        with pytest.raises(IndexError):
            so.llm_to_rvq(np.array(case), 2)
        so.llm_to_rvq(np.array(case), 2, safe=False)  # no raise


def test_encoder_inputs_bruteforce():
    c = so.SystemConfig()
    rng = np.random.default_rng(0)
    ctx = rng.integers(0, 1024, size=(250, 16)).astype(np.int32)
    ctx[:7] = -1                 # empty slots of a fresh stream -> MASK
    ctx[100, 2] = -1
    style = 17410 + np.arange(6) * 1024 + rng.integers(0, 1024, 6)
    got = so.build_encoder_inputs_host(ctx, c, style)
    assert got.shape == (2, 1006) and got.dtype == np.int32
    for f in range(250):
        for d in range(4):
            v = ctx[f, d]
            exp = 1 if v < 0 else 2 + 1024 * d + v
            assert got[0, f * 4 + d] == exp and got[1, f * 4 + d] == exp
    assert got[0, 1000:].tolist() == style.tolist()
    assert got[1, 1000:].tolist() == [1] * 6
    unc = so.build_encoder_inputs_host(ctx, c, None)
    assert unc[0, 1000:].tolist() == [1] * 6


def test_context_roll():
    rng = np.random.default_rng(1)
    ctx = rng.integers(-1, 1024, size=(250, 16)).astype(np.int32)
    new = rng.integers(0, 1024, size=(50, 16)).astype(np.int32)
    got = so.roll_context(ctx, new)
    np.testing.assert_array_equal(got[:200], ctx[50:])
    np.testing.assert_array_equal(got[200:], new)


def test_codec_input_frames():
    """system.cpp:294-313: [clamped last context row | chunk ids]; zeros on chunk 0."""
    from oracle import system_oracle as SO
    ctx = np.arange(5 * 3).reshape(5, 3).astype(np.int32) - 2  # last row 10..12, first row has -2, -1
    ctx[-1, 0] = -1
    new = np.full((2, 3), 7, np.int32)
    a = SO.codec_input_frames(ctx, new, chunk_index=3)
    np.testing.assert_array_equal(a, [[0, 11, 12], [7, 7, 7], [7, 7, 7]])
    b = SO.codec_input_frames(ctx, new, chunk_index=0)
    np.testing.assert_array_equal(b[0], [0, 0, 0])


def test_crossfade_equal_power():
    """Ramp sin(t pi/2) in, sin((1-t) pi/2) out: at t = 0 the old tail alone,
    at t = 1 the new audio alone, and fin^2 + fout^2 = 1 (equal power), so a
    constant signal faded against itself keeps its power profile."""
    from oracle import system_oracle as SO
    xf = 5
    wave = np.ones((12, 2), np.float32) * 2.0
    tail = np.full((xf, 2), 3.0, np.float32)
    dec, nxt = SO.crossfade_chunk(wave, tail, chunk_index=1, xf_samples=xf)
    assert dec.shape == (7, 2) and nxt.shape == (xf, 2)
    np.testing.assert_allclose(dec[0], [3.0, 3.0], rtol=1e-6)
    np.testing.assert_allclose(dec[xf - 1], [2.0, 2.0], rtol=1e-6)
    t = np.arange(xf) / (xf - 1)
    np.testing.assert_allclose(dec[:xf, 0], 2 * np.sin(t * np.pi / 2) + 3 * np.cos(t * np.pi / 2), rtol=1e-5)
    np.testing.assert_array_equal(dec[xf:], wave[xf:7])
    dec0, _ = SO.crossfade_chunk(wave, tail, chunk_index=0, xf_samples=xf)
    np.testing.assert_array_equal(dec0, wave[:7])
