"""Pins of the codec oracle (RVQ dequantisation, SpectroStream decoder, iSTFT):
an independent library (torch.nn.functional, float64), brute-force loops,
closed forms and the STFT round trip, plus the two identities the HIP codec's
design relies on (phase-split transposed conv, shortcut before repeat)."""

from __future__ import annotations

import math

import numpy as np
import pytest

import synth_bundle
from oracle import codec_oracle as C


def _torch():
    return pytest.importorskip("torch")


@pytest.mark.parametrize("k,s", [((3, 3), (1, 1)), ((1, 1), (1, 1)), ((7, 7), (1, 1)), ((3, 4), (1, 2)),
                                 ((4, 3), (2, 1))])
def test_conv2d_matches_torch(k, s):
    torch = _torch()
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 9, 11, 5))
    w = rng.standard_normal((6, 5) + k)
    b = rng.standard_normal(6)
    got = C.conv2d(x, w, b, s)
    ref = torch.nn.functional.conv2d(torch.from_numpy(x).permute(0, 3, 1, 2), torch.from_numpy(w),
                                     torch.from_numpy(b), stride=s).permute(0, 2, 3, 1).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("k,s", [((4, 3), (2, 1)), ((4, 4), (2, 2)), ((3, 4), (1, 2)), ((3, 6), (1, 3))])
def test_conv_transpose2d_matches_torch(k, s):
    torch = _torch()
    rng = np.random.default_rng(2)
    x = rng.standard_normal((2, 4, 5, 3))
    w = rng.standard_normal((3, 4) + k)  # stored (in, out, kH, kW)
    b = rng.standard_normal(4)
    got = C.conv_transpose2d(x, w, b, s)
    ref = torch.nn.functional.conv_transpose2d(torch.from_numpy(x).permute(0, 3, 1, 2), torch.from_numpy(w),
                                               torch.from_numpy(b), stride=s).permute(0, 2, 3, 1).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
    assert got.shape[1:3] == ((4 - 1) * s[0] + k[0], (5 - 1) * s[1] + k[1])


def test_conv_transpose2d_brute_force():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((1, 2, 3, 2))
    w = rng.standard_normal((2, 3, 3, 4))
    s = (1, 3)
    got = C.conv_transpose2d(x, w, None, s)
    Ho, Wo = (2 - 1) * 1 + 3, (3 - 1) * 3 + 4
    ref = np.zeros((1, Ho, Wo, 3))
    for h in range(2):
        for ww in range(3):
            for i in range(2):
                for o in range(3):
                    for kh in range(3):
                        for kw in range(4):
                            ref[0, h * s[0] + kh, ww * s[1] + kw, o] += x[0, h, ww, i] * w[i, o, kh, kw]
    np.testing.assert_allclose(got, ref, rtol=1e-13, atol=1e-13)


def test_pads_closed_form():
    # causal: top = kH - sH, width split floor/ceil of (kW - 1) at stride 1
    assert C.causal_pads((3, 3), (1, 1), 5) == (2, 1, 1)
    assert C.causal_pads((7, 7), (1, 1), 480) == (6, 3, 3)
    assert C.causal_pads((3, 4), (1, 2), 10) == (2, 1, 1)
    x = np.ones((1, 4, 5, 2))
    y = C.same_pad(x, (3, 3), (1, 1))
    assert y.shape == (1, 6, 7, 2) and y[0, 0].sum() == 0 and y[0, 1, 1:6].sum() == 10


def test_elu_closed_form():
    x = np.array([-3.0, -0.5, 0.0, 0.25, 4.0], dtype=np.float32)
    np.testing.assert_allclose(C.elu(x), [math.exp(-3) - 1, math.exp(-0.5) - 1, 0.0, 0.25, 4.0], rtol=1e-6)


def test_rvq_dequantization_brute_force_and_one_hot():
    rng = np.random.default_rng(4)
    cb = rng.standard_normal((20, 8, 5)).astype(np.float32)
    tok = rng.integers(0, 8, size=(6, 16))
    got = C.rvq_dequantization(tok, cb)
    ref = np.zeros((6, 5), np.float32)
    for n in range(6):
        for k in range(16):
            ref[n] = ref[n] + cb[k, tok[n, k]]
    np.testing.assert_array_equal(got, ref)
    # one-hot codebooks: level k, code c -> e_c * 10^k
    oh = np.zeros((3, 4, 4), np.float32)
    for k in range(3):
        for c in range(4):
            oh[k, c, c] = 10.0 ** k
    v = C.rvq_dequantization(np.array([[1, 1, 3]]), oh)
    np.testing.assert_array_equal(v, [[0, 11, 0, 100]])
    with pytest.raises(ValueError):
        C.rvq_dequantization(np.zeros(3, np.int64), cb)


def _brute_istft(spec, T, N=960, hop=480):
    B, H, F, _ = spec.shape
    out = np.zeros((B, T, 2))
    t = np.arange(N)
    win = 0.5 - 0.5 * np.cos(2 * math.pi * t / N)
    per = (win ** 2).reshape(2, hop).sum(0)
    syn = win / np.concatenate([per, per])
    for b in range(B):
        for s in range(2):
            frames = np.zeros((H, N))
            for i in range(H):
                re = spec[b, i, :, 2 * s]
                im = spec[b, i, :, 2 * s + 1]
                x = np.full(N, re[0])
                for k in range(1, F):
                    x += 2 * (re[k] * np.cos(2 * math.pi * k * t / N) - im[k] * np.sin(2 * math.pi * k * t / N))
                frames[i] = x / N * syn
            audio = np.zeros((H + 1) * hop)
            for i in range(H):
                audio[i * hop:i * hop + N] += frames[i]
            out[b, :, s] = audio[:T]
    return out


def test_istft_brute_force():
    rng = np.random.default_rng(5)
    spec = rng.standard_normal((1, 3, 480, 4))
    T = 3 * 480 + 200
    got = C.istft_postprocess(spec, 1, T)
    np.testing.assert_allclose(got, _brute_istft(spec, T), rtol=1e-9, atol=1e-10)
    assert got.shape == (1, T, 2)


def test_istft_round_trip():
    """Hann analysis frames at hop 480 -> rfft (Nyquist dropped) -> istft
    reconstructs the signal from the second hop on: the synthesis window is
    hann / sum(hann^2) over the two phases, so each sample's two
    contributions sum to 1."""
    N, hop, H = 960, 480, 8
    t = np.arange((H + 1) * hop)
    x = np.stack([np.sin(2 * math.pi * 440 * t / 48000) + 0.3 * np.cos(2 * math.pi * 3100 * t / 48000),
                  0.5 * np.sin(2 * math.pi * 1234 * t / 48000 + 0.4)], axis=-1)
    win = 0.5 - 0.5 * np.cos(2 * math.pi * np.arange(N) / N)
    spec = np.zeros((1, H, 480, 4))
    for s in range(2):
        for i in range(H):
            X = np.fft.rfft(x[i * hop:i * hop + N, s] * win)
            spec[0, i, :, 2 * s] = X[:480].real
            spec[0, i, :, 2 * s + 1] = X[:480].imag
    y = C.istft_postprocess(spec, 1, H * hop)
    np.testing.assert_allclose(y[0, hop:H * hop], x[hop:H * hop], atol=1e-9)


def test_decoder_shapes_and_finite():
    cfg = C.CodecConfig.tiny()
    shape = synth_bundle.CodecShape.tiny()
    assert shape.channels() == (cfg.embedding_dim, cfg.proj_ch, [b.in_ch for b in cfg.blocks],
                                [b.out_ch for b in cfg.blocks])
    w = synth_bundle.make_codec_weights(shape, levels=16, codebook=64)
    o = C.OracleCodec(w, cfg, "fp64")
    S = 3
    tok = np.random.default_rng(6).integers(0, 64, size=(S, 16))
    rec = {}
    audio = o.decode(tok, rec)
    assert rec["spec_planar"].shape == (2, 4 * S, 480, 2)  # H = 4 (S + 1) - 4
    assert rec["block0"].shape == (2, 2 * (S + 1), 5, cfg.blocks[0].out_ch // 2)
    assert audio.shape == (S * 1920, 2) and np.isfinite(audio).all()
    for name, shp in synth_bundle.codec_layout(shape):
        assert w[name].shape == shp


def test_package_codec_shape_is_the_oracle_config():
    ref, sh = C.CodecConfig.reference(), synth_bundle.CodecShape.reference()
    for a, b in zip(ref.blocks, sh.blocks):
        assert (a.in_ch, a.out_ch, a.stride, a.transpose_kernel, a.post_kernel) == \
            (b.in_ch, b.out_ch, b.stride, b.transpose_kernel, b.post_kernel)
    assert (ref.embedding_dim, ref.proj_ch, ref.unfold) == (sh.embedding_dim, sh.proj_ch, sh.unfold)


def test_flops_table():
    fl = synth_bundle.codec_flops(synth_bundle.CodecShape.reference(), 51)
    assert 195e9 < fl["total"] < 205e9


def test_design_identity_shortcut_commutes_with_repeat():
    """1x1 conv of the repeated input == repeat of the 1x1 conv (the HIP codec
    applies a block's shortcut on the input grid)."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal((2, 3, 4, 5))
    w = rng.standard_normal((6, 5, 1, 1))
    b = rng.standard_normal(6)
    rep = np.repeat(np.repeat(x, 2, axis=1), 3, axis=2)
    a = C.conv2d(rep, w, b)
    c = np.repeat(np.repeat(C.conv2d(x, w, b), 2, axis=1), 3, axis=2)
    np.testing.assert_allclose(a, c, rtol=1e-13)


@pytest.mark.parametrize("bi", range(7))
def test_design_identity_phase_split(bi):
    """A transposed conv with the reference's crop equals, per output phase
    (oy % sH, (ox + crop_w_start) % sW), a stride-1 conv over the input with
    taps (kh, kw) = (ph + sH * j, pw + sW * i) reading x[q_y - j, q_x - i] --
    the decomposition the HIP codec launches (one sub-problem per phase)."""
    blk = C.CodecConfig.reference().blocks[bi]
    rng = np.random.default_rng(8 + bi)
    H, W, Ci, Co = 4, 5, 3, 2
    x = rng.standard_normal((1, H, W, Ci))
    w = rng.standard_normal((Ci, Co) + blk.transpose_kernel)
    kh, kw = blk.transpose_kernel
    sh, sw = blk.stride
    full = C.conv_transpose2d(x, w, None, blk.stride)
    ch = kh - sh
    cs = (kw - sw) // 2
    ce = (kw - sw) - cs
    ref = full[:, :full.shape[1] - ch, cs:full.shape[2] - ce]
    Hc, Wc = ref.shape[1], ref.shape[2]
    got = np.full_like(ref, np.nan)
    for ph in range(sh):
        for pw in range(sw):
            # output (oy, ox) = (qy * sh + ph, qx * sw + pw - cs), qx from qx0
            qx0 = -(-(cs - pw) // sw) if cs > pw else 0
            gy = -(-(Hc - ph) // sh)
            gx = -(-(Wc - (qx0 * sw + pw - cs)) // sw)
            for a in range(gy):
                for bb in range(gx):
                    oy, ox = a * sh + ph, (bb + qx0) * sw + pw - cs
                    if oy >= Hc or ox >= Wc:
                        continue
                    acc = np.zeros(Co)
                    for j in range((kh - ph + sh - 1) // sh):
                        for i in range((kw - pw + sw - 1) // sw):
                            iy, ix = a - j, bb + qx0 - i
                            if 0 <= iy < H and 0 <= ix < W:
                                acc += x[0, iy, ix] @ w[:, :, ph + sh * j, pw + sw * i]
                    got[0, oy, ox] = acc
    assert not np.isnan(got).any()
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
