"""CPU restatement of the reference's integer token plumbing around the decode path.

TEST INFRASTRUCTURE ONLY (see depthformer_oracle.py header).

Restates:
  * vocabulary layout constants        -- system.h:44-83
  * build_encoder_inputs_host          -- system.cpp:62-95
  * build_vocab_masks (level ranges)   -- system.cpp:135-157
  * rvq_to_llm / llm_to_rvq            -- rvq.cpp:105-132 (upstream utils.py:106-147)
  * context roll after a chunk         -- system.cpp:320-333
  * codec input + crossfade of a chunk -- system.cpp:294-313, 395-440
Pinned by the upstream known answers (system_test.py:29-41, decode_test.py:26-71,
utils_test.py:99-149) restated in tests/test_oracle_system.py; the crossfade
by its closed form (equal-power sine ramp) in the same file.
"""

from __future__ import annotations

import dataclasses
from typing import Optional, Sequence

import numpy as np


@dataclasses.dataclass(frozen=True)
class SystemConfig:
    """system.h:44-83."""

    chunk_length: float = 2.0
    context_length: float = 10.0
    codec_frame_rate: float = 25.0
    codec_rvq_codebook_size: int = 1024
    style_rvq_codebook_size: int = 1024
    encoder_codec_rvq_depth: int = 4
    encoder_style_rvq_depth: int = 6
    decoder_codec_rvq_depth: int = 16
    llm_vocab_size: int = 29824

    def chunk_length_frames(self) -> int:
        return int(self.chunk_length * self.codec_frame_rate + 0.5)

    def context_length_frames(self) -> int:
        return int(self.context_length * self.codec_frame_rate + 0.5)

    def vocab_mask_token(self) -> int:
        return 1

    def vocab_codec_offset(self) -> int:
        return 2

    def vocab_codec_size(self) -> int:
        return self.decoder_codec_rvq_depth * self.codec_rvq_codebook_size

    def vocab_style_offset(self) -> int:
        return self.vocab_codec_offset() + self.vocab_codec_size() + 1024

    def encoder_length(self) -> int:
        return (self.context_length_frames() * self.encoder_codec_rvq_depth
                + self.encoder_style_rvq_depth)


def build_encoder_inputs_host(context_tokens: np.ndarray, cfg: SystemConfig,
                              style_tokens: Optional[Sequence[int]]) -> np.ndarray:
    """system.cpp:62-95 -> (2, enc_len) int32.

    Row 0: codec context levels 0..enc_depth-1 mapped to ``2 + 1024 d + v``
    (MASK for v < 0), followed by the style ids; row 1: same codec block,
    style replaced by MASK.  ``style_tokens is None`` means unconditioned
    (system.cpp:200-210: every style slot MASK).
    """
    ctx = np.asarray(context_tokens, dtype=np.int32)
    frames, depth = ctx.shape
    e, s = cfg.encoder_codec_rvq_depth, cfg.encoder_style_rvq_depth
    mask = cfg.vocab_mask_token()
    enc_len = frames * e + s
    out = np.empty((2, enc_len), dtype=np.int32)
    lvl = np.arange(e, dtype=np.int32)[None, :]
    v = ctx[:, :e]
    codec = np.where(v >= 0, cfg.vocab_codec_offset() + lvl * cfg.codec_rvq_codebook_size + v, mask)
    out[0, :frames * e] = codec.reshape(-1)
    style = np.full((s,), mask, dtype=np.int32) if style_tokens is None else np.asarray(style_tokens, dtype=np.int32)
    if style.shape != (s,):
        raise ValueError("style_tokens size != encoder_style_rvq_depth")
    out[0, frames * e:] = style
    out[1, :frames * e] = out[0, :frames * e]
    out[1, frames * e:] = mask
    return out


def vocab_level_range(cfg: SystemConfig, level: int):
    """system.cpp:135-157: level keeps [2 + C*level, 2 + C*(level+1))."""
    start = cfg.vocab_codec_offset() + level * cfg.codec_rvq_codebook_size
    return start, start + cfg.codec_rvq_codebook_size


def build_vocab_masks(cfg: SystemConfig) -> np.ndarray:
    """(depth, vocab) bool masks of system.cpp:135-157."""
    m = np.zeros((cfg.decoder_codec_rvq_depth, cfg.llm_vocab_size), dtype=bool)
    for lvl in range(cfg.decoder_codec_rvq_depth):
        a, b = vocab_level_range(cfg, lvl)
        m[lvl, a:b] = True
    return m


def rvq_to_llm(tokens: np.ndarray, codebook_size: int, offset: int = 0) -> np.ndarray:
    """rvq.cpp:105-110 (range checks of upstream utils.py:110-113)."""
    t = np.asarray(tokens)
    if t.ndim == 0:
        raise ValueError(f"Invalid array shape: {t.shape}")
    if np.any(t < 0) or np.any(t >= codebook_size):
        raise IndexError(f"Invalid array values: {t}")
    depth = t.shape[-1]
    lv = (np.arange(depth) * codebook_size).reshape(*([1] * (t.ndim - 1) + [depth]))
    return (t + offset + lv).astype(np.int32)


def llm_to_rvq(tokens: np.ndarray, codebook_size: int, offset: int = 0,
               safe: bool = True) -> np.ndarray:
    """rvq.cpp:112-132 / upstream utils.py:123-147 (safe -> IndexError; the C++ raises
    std::invalid_argument on exactly the same ids: floor((t - offset) / C) != level)."""
    t = np.asarray(tokens)
    if t.ndim == 0:
        raise ValueError(f"Invalid array shape: {t.shape}")
    depth = t.shape[-1]
    r = np.maximum(t - offset, 0)
    subset = r // codebook_size
    exp = np.arange(depth).reshape(*([1] * (t.ndim - 1) + [depth]))
    bad = int(np.logical_or(t < offset, subset != exp).sum())
    if bad and safe:
        raise IndexError(f"{bad}/{t.size} invalid tokens")
    return (r % codebook_size).astype(np.int32)


def roll_context(context_tokens: np.ndarray, new_rvq: np.ndarray) -> np.ndarray:
    """system.cpp:320-333: drop the oldest chunk_frames rows, append the new RVQ ids."""
    ctx = np.asarray(context_tokens, dtype=np.int32)
    new = np.asarray(new_rvq, dtype=np.int32)
    frames = ctx.shape[0]
    n = new.shape[0]
    out = np.empty_like(ctx)
    src = (np.arange(frames) + n) % frames
    out[:] = ctx[src]
    out[frames - n:] = new
    return out


def codec_input_frames(context_before: np.ndarray, chunk_rvq: np.ndarray, chunk_index: int,
                       xf_frames: int = 1) -> np.ndarray:
    """system.cpp:294-313: the decoder input of a chunk: the context's last
    xf_frames rows before the roll (negative ids clamped to 0; zeros on chunk
    0), then the chunk's RVQ ids."""
    ctx = np.asarray(context_before, dtype=np.int32)
    levels = ctx.shape[1]
    xf = np.zeros((xf_frames, levels), np.int32)
    if chunk_index > 0:
        xf = np.maximum(ctx[ctx.shape[0] - xf_frames:], 0).astype(np.int32)
    return np.concatenate([xf, np.asarray(chunk_rvq, dtype=np.int32)], axis=0)


def crossfade_chunk(wave: np.ndarray, prev_tail: Optional[np.ndarray], chunk_index: int, xf_samples: int = 1920):
    """system.cpp:395-440: (decoded, next_tail) from the chunk's waveform (T, C):
    the last xf_samples samples become the next tail; the rest is the chunk's
    audio, its first xf_samples ramped in (sin) against the previous tail
    ramped out (sin of the complement), t = i / (xf_samples - 1), in float32."""
    wave = np.asarray(wave, dtype=np.float32)
    T = wave.shape[0]
    nxt = wave[T - xf_samples:].copy()
    dec = wave[:T - xf_samples].copy()
    if chunk_index > 0 and prev_tail is not None and prev_tail.shape[0] == xf_samples and dec.shape[0] >= xf_samples:
        t = np.arange(xf_samples, dtype=np.float32) / np.float32(max(xf_samples - 1, 1))
        fin = np.sin(t * np.float32(1.5707963267948966)).astype(np.float32)
        fout = np.sin((np.float32(1.0) - t) * np.float32(1.5707963267948966)).astype(np.float32)
        dec[:xf_samples] = dec[:xf_samples] * fin[:, None] + prev_tail * fout[:, None]
    return dec, nxt
