"""CPU restatement (numpy) of the reference's codec decode: RVQ dequantisation,
the SpectroStream decoder and the iSTFT post-processor.

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module: it is
the checker the HIP codec is compared against.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it.

Reference files (paths relative to ``src/magenta_realtime_mlx/``):
  * rvq_dequantization             rvq.cpp:68-88
  * elu                            nn_ops.h:31-39
  * causal_same_pad / same_pad     spectrostream.cpp:41-85
  * unfold_width                   spectrostream.cpp:95-102
  * WNConv2d / WNConvTranspose2d   spectrostream.cpp:110-158
  * Res1x1Block / Res3x3Block      spectrostream.cpp:163-200
  * DecoderResBlock                spectrostream.cpp:202-262
  * block table, decoder forward   spectrostream.cpp:328-432
  * istft_postprocess              spectrostream.cpp:593-681
  * the codec call site            system.cpp:373-390 (decoder in fp32,
                                   system.cpp:118-119)

Layouts follow the reference: activations NHWC (B, H, W, C); stored conv
weights (out, in, kH, kW); stored transposed-conv weights (in, out, kH, kW)
(the transposes at spectrostream.cpp:110-116 give MLX's (out, kH, kW, in)).
MLX's ``conv2d`` is a cross-correlation without padding; its
``conv_transpose2d`` with padding 0 is the adjoint of that convolution:
out[h*s + kh, w*s + kw, o] += x[h, w, i] * W[i, o, kh, kw], output size
(H - 1) * s + kH (the same definition as torch's ``conv_transpose2d``).

How each part is pinned (tests/test_oracle_codec.py):
  * conv2d, conv_transpose2d     -- torch.nn.functional (an independent
                                    library, float64) and brute-force loops;
  * pads                         -- closed forms at the shapes the decoder uses;
  * decoder shape arithmetic     -- the header's (B, H, 480, 4) output and
                                    H = 4 * (S + 1) - 4;
Bundle layout, synthetic weights and FLOP counts are the package's
(synth_bundle.codec_layout / make_codec_weights / codec_flops).
  * istft_postprocess            -- a brute-force DFT + overlap-add loop, and
                                    the round trip istft(stft_hann(x)) == x
                                    (Hann analysis window, the reference's
                                    Hann / sum-of-squares synthesis window);
  * rvq_dequantization           -- a brute-force loop and one-hot codebooks;
  * the GPU design's identities  -- 1x1 conv commutes with the residual
                                    repeat; a transposed conv equals the sum
                                    of its stride phases, each a stride-1
                                    conv over the input.
Parity unpinned: MLX's exact fp32 accumulation order inside conv / FFT (the
GPU is compared within a tolerance).
"""

from __future__ import annotations

import dataclasses
import math
from typing import Dict, List, Tuple

import numpy as np

# ---------------------------------------------------------------------------
# Configuration (spectrostream.cpp:328-362, system.h:44-83)


@dataclasses.dataclass(frozen=True)
class DecBlock:
    in_ch: int
    out_ch: int
    stride: Tuple[int, int]
    transpose_kernel: Tuple[int, int]
    post_kernel: Tuple[int, int]


@dataclasses.dataclass(frozen=True)
class CodecConfig:
    embedding_dim: int = 256          # SpectroStreamDecoder::kEmbeddingDim
    proj_ch: int = 2560               # input_proj 256 -> 2560 -> 2560
    unfold: int = 5                   # unfold_width(x, 5): 2560 = 5 x 512
    blocks: Tuple[DecBlock, ...] = (
        DecBlock(512, 1024, (2, 1), (4, 3), (3, 3)),
        DecBlock(512, 256, (2, 2), (4, 4), (3, 3)),
        DecBlock(256, 256, (1, 2), (3, 4), (3, 3)),
        DecBlock(256, 256, (1, 2), (3, 4), (3, 3)),
        DecBlock(256, 128, (1, 3), (3, 6), (3, 3)),
        DecBlock(128, 128, (1, 2), (3, 4), (3, 3)),
        DecBlock(128, 64, (1, 2), (3, 4), (3, 3)),
    )
    out_ch: int = 2                   # output_conv 7x7 -> (real, imag)
    out_kernel: Tuple[int, int] = (7, 7)
    temporal_pad: int = 1             # kTemporalPad
    temporal_crop: int = 4            # kTemporalCrop
    n_fft: int = 960
    hop: int = 480
    samples_per_frame: int = 1920     # codec_sample_rate / codec_frame_rate

    @property
    def input_conv_ch(self) -> int:
        return self.proj_ch // self.unfold

    @staticmethod
    def reference() -> "CodecConfig":
        return CodecConfig()

    @staticmethod
    def tiny() -> "CodecConfig":
        """Channel counts / 4 (test-only): same strides, kernels, crops and
        frequency axis, so every index path of the full decoder is exercised."""
        r = CodecConfig()
        return dataclasses.replace(
            r, embedding_dim=64, proj_ch=640,
            blocks=tuple(DecBlock(b.in_ch // 4, b.out_ch // 4, b.stride, b.transpose_kernel, b.post_kernel)
                         for b in r.blocks))


# ---------------------------------------------------------------------------
# RVQ (rvq.cpp:68-88)


def rvq_dequantization(tokens: np.ndarray, codebooks: np.ndarray) -> np.ndarray:
    """rvq.cpp:68-88: vectors = sum over levels k < K of codebooks[k][tokens[:, k]],
    accumulated in float32 from zeros, level by level."""
    tokens = np.asarray(tokens)
    if codebooks.ndim != 3:
        raise ValueError("rvq_dequantization: codebooks must be (K, C, D)")
    if tokens.ndim != 2:
        raise ValueError("rvq_dequantization: tokens must be (N, K)")
    n, K = tokens.shape
    out = np.zeros((n, codebooks.shape[2]), dtype=np.float32)
    for k in range(K):
        out = out + codebooks[k][tokens[:, k]].astype(np.float32)
    return out


# ---------------------------------------------------------------------------
# Elementwise and padding (nn_ops.h:31-39, spectrostream.cpp:41-102)


def elu(x: np.ndarray) -> np.ndarray:
    """nn_ops.h:31-39: where(x > 0, x, exp(x) - 1) (alpha 1)."""
    one = x.dtype.type(1.0)
    return np.where(x > 0, x, np.exp(np.minimum(x, 0)) - one).astype(x.dtype)


def causal_pads(kernel: Tuple[int, int], stride: Tuple[int, int], iw: int) -> Tuple[int, int, int]:
    """spectrostream.cpp:41-62: (top, left, right); nothing at the bottom."""
    kh, kw = kernel
    sh, sw = stride
    ow = -(-iw // sw)
    tot = max((ow - 1) * sw + kw - iw, 0)
    return kh - sh, tot // 2, tot - tot // 2


def causal_same_pad(x, kernel, stride):
    top, left, right = causal_pads(kernel, stride, x.shape[2])
    return np.pad(x, ((0, 0), (max(top, 0), 0), (left, right), (0, 0)))


def same_pad(x, kernel, stride):
    """spectrostream.cpp:64-85."""
    ih, iw = x.shape[1], x.shape[2]
    kh, kw = kernel
    sh, sw = stride
    ph = max((-(-ih // sh) - 1) * sh + kh - ih, 0)
    pw = max((-(-iw // sw) - 1) * sw + kw - iw, 0)
    return np.pad(x, ((0, 0), (ph // 2, ph - ph // 2), (pw // 2, pw - pw // 2), (0, 0)))


def unfold_width(x, f):
    """spectrostream.cpp:95-102: (B, H, W, C*f) -> (B, H, W*f, C), a reshape."""
    B, H, W, C = x.shape
    return x.reshape(B, H, W * f, C // f)


# ---------------------------------------------------------------------------
# Convolutions (spectrostream.cpp:110-158)


def conv2d(x: np.ndarray, w: np.ndarray, b, stride=(1, 1)) -> np.ndarray:
    """WNConv2d (spectrostream.cpp:135-139): valid cross-correlation of NHWC x
    with stored weights (O, I, kH, kW), plus bias."""
    B, H, W, Ci = x.shape
    O, I, kh, kw = w.shape
    assert I == Ci, (I, Ci)
    sh, sw = stride
    Ho = (H - kh) // sh + 1
    Wo = (W - kw) // sw + 1
    out = np.zeros((B, Ho, Wo, O), dtype=x.dtype)
    for i in range(kh):
        for j in range(kw):
            xs = x[:, i:i + sh * (Ho - 1) + 1:sh, j:j + sw * (Wo - 1) + 1:sw, :]
            out += xs @ w[:, :, i, j].T.astype(x.dtype)
    if b is not None:
        out += b.astype(x.dtype)
    return out


def conv_transpose2d(x: np.ndarray, w: np.ndarray, b, stride) -> np.ndarray:
    """WNConvTranspose2d (spectrostream.cpp:153-158): stored weights (I, O, kH,
    kW); out[h*sh + i, w*sw + j] += x[h, w] @ W[:, :, i, j]; size (H-1)*s + k."""
    B, H, W, Ci = x.shape
    I, O, kh, kw = w.shape
    assert I == Ci, (I, Ci)
    sh, sw = stride
    Ho, Wo = (H - 1) * sh + kh, (W - 1) * sw + kw
    out = np.zeros((B, Ho, Wo, O), dtype=x.dtype)
    for i in range(kh):
        for j in range(kw):
            out[:, i:i + sh * (H - 1) + 1:sh, j:j + sw * (W - 1) + 1:sw, :] += x @ w[:, :, i, j].astype(x.dtype)
    if b is not None:
        out += b.astype(x.dtype)
    return out


# ---------------------------------------------------------------------------
# Blocks (spectrostream.cpp:163-262)


class OracleCodec:
    """SpectroStreamDecoder + rvq_dequantization + istft_postprocess.

    ``weights``: decoder bundle (name -> fp32 array, stored layouts) plus
    ``codebooks`` (K, C, D).  ``mode``: "fp32" (the reference's codec dtype,
    system.cpp:118-119) or "fp64"."""

    def __init__(self, weights: Dict[str, np.ndarray], cfg: CodecConfig, mode: str = "fp32"):
        self.cfg = cfg
        self.dt = np.float32 if mode == "fp32" else np.float64
        self.w = {k: np.asarray(v, dtype=self.dt) for k, v in weights.items()}

    def _c(self, name, x, stride=(1, 1)):
        return conv2d(x, self.w[name + ".weight"], self.w.get(name + ".bias"), stride)

    def res1x1(self, p, x, pre_elu=False):
        """spectrostream.cpp:174-181."""
        skip = self._c(p + ".shortcut", x)
        m = elu(x) if pre_elu else x
        m = self._c(p + ".conv1", m)
        m = elu(m)
        m = self._c(p + ".conv2", m)
        return m + skip

    def res3x3(self, p, x, causal=True):
        """spectrostream.cpp:191-200."""
        pad = causal_same_pad if causal else same_pad
        y = elu(x)
        y = self._c(p + ".conv1", pad(y, (3, 3), (1, 1)))
        y = elu(y)
        y = self._c(p + ".conv2", pad(y, (3, 3), (1, 1)))
        return y + x

    def dec_block(self, i, x):
        """spectrostream.cpp:224-262."""
        b = self.cfg.blocks[i]
        p = f"decoder_blocks.{i}"
        kh, kw = b.transpose_kernel
        sh, sw = b.stride
        crop_h = kh - sh
        cws = (kw - sw) // 2
        cwe = (kw - sw) - cws
        residual = x
        y = elu(x)
        y = conv_transpose2d(y, self.w[p + ".conv_transpose.weight"], self.w[p + ".conv_transpose.bias"], b.stride)
        if crop_h > 0:
            y = y[:, :y.shape[1] - crop_h]
        if cws > 0 or cwe > 0:
            y = y[:, :, cws:y.shape[2] - cwe]
        y = elu(y)
        y = self._c(p + ".conv", causal_same_pad(y, b.post_kernel, (1, 1)))
        H, W = residual.shape[1], residual.shape[2]
        if sh != 1:
            residual = np.repeat(residual, sh, axis=1)[:, :H * sh]
        if sw != 1:
            residual = np.repeat(residual, sw, axis=2)[:, :, :W * sw]
        if b.in_ch != b.out_ch:
            residual = self._c(p + ".shortcut", residual)
        return y + residual

    def decoder(self, emb: np.ndarray, record: Dict | None = None) -> np.ndarray:
        """spectrostream.cpp:365-432: (B, S, E) -> (B, H, 480, 4) with the last
        axis [s0_re, s0_im, s1_re, s1_im]."""
        cfg = self.cfg
        B, S, E = emb.shape
        x = np.concatenate([emb.astype(self.dt), np.zeros((B, cfg.temporal_pad, E), self.dt)], axis=1)
        x = x[:, :, None, :]
        x = self.res1x1("input_proj", x)
        x = unfold_width(x, cfg.unfold)
        x = self.res3x3("input_conv", x, causal=True)
        if record is not None:
            record["input_conv"] = x.copy()
        x = self.dec_block(0, x)
        Bn, H, W, C = x.shape
        x = x.reshape(Bn, H, W, 2, C // 2).transpose(3, 0, 1, 2, 4).reshape(2 * Bn, H, W, C // 2)
        if record is not None:
            record["block0"] = x.copy()
        for i in range(1, len(cfg.blocks)):
            x = self.dec_block(i, x)
            if record is not None:
                record[f"block{i}"] = x.copy()
        x = elu(x)
        x = self._c("output_conv", causal_same_pad(x, cfg.out_kernel, (1, 1)))
        x = x[:, cfg.temporal_crop:]
        if record is not None:
            record["spec_planar"] = x.copy()  # (2B, H, 480, 2)
        H2, W2, C2 = x.shape[1:]
        x = x.reshape(2, B, H2, W2, C2).transpose(1, 2, 3, 0, 4).reshape(B, H2, W2, 2 * C2)
        return x

    def decode(self, rvq_tokens: np.ndarray, record: Dict | None = None) -> np.ndarray:
        """system.cpp:373-390: tokens (S, K) -> audio (S * 1920, 2) float32."""
        emb = rvq_dequantization(rvq_tokens, self.w["codebooks"].astype(np.float32))
        if record is not None:
            record["embeddings"] = emb.copy()
        spec = self.decoder(emb[None], record)
        T = rvq_tokens.shape[0] * self.cfg.samples_per_frame
        return istft_postprocess(spec, 1, T, self.cfg)[0].astype(np.float32)


# ---------------------------------------------------------------------------
# iSTFT (spectrostream.cpp:593-681)


def synthesis_window(n_fft: int = 960, hop: int = 480, dtype=np.float32) -> np.ndarray:
    """spectrostream.cpp:636-646: hann / (sum of hann^2 over the two hop phases)."""
    t = np.arange(n_fft, dtype=dtype)
    win = dtype(0.5) - dtype(0.5) * np.cos(t * dtype(2.0 * math.pi / n_fft))
    sq = win * win
    periodic = sq.reshape(2, hop).sum(axis=0)
    return (win / np.concatenate([periodic, periodic])).astype(dtype)


def istft_postprocess(spec: np.ndarray, B: int, target_length: int, cfg: CodecConfig = CodecConfig()) -> np.ndarray:
    """spectrostream.cpp:593-681: (B, H, 480, 4) -> (B, target_length, 2)."""
    N, hop = cfg.n_fft, cfg.hop
    dt = np.float64 if spec.dtype == np.float64 else np.float32
    frames, freq = spec.shape[1], spec.shape[2]
    x = np.pad(spec, ((0, 0), (0, 0), (0, 1), (0, 0))).reshape(B, frames, freq + 1, 2, 2)
    xc = x[..., 0] + 1j * x[..., 1]                       # (B, H, 481, 2)
    xc = xc.transpose(0, 3, 1, 2).reshape(B * 2, frames, freq + 1)
    tf = np.fft.irfft(xc, n=N, axis=-1).astype(dt)
    wf = tf * synthesis_window(N, hop, dt)[None, None, :]
    left, right = wf[:, :, :hop], wf[:, :, hop:]
    body = left.copy()
    body[:, 1:] += right[:, :-1]
    audio = np.concatenate([body.reshape(B * 2, frames * hop), right[:, -1]], axis=-1)
    audio = audio[:, :target_length].reshape(B, 2, target_length).transpose(0, 2, 1)
    return np.ascontiguousarray(audio)
