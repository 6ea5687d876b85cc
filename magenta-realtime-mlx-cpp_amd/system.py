"""Host-side token plumbing around the decode path (the LLM half of System::generate_chunk).

* ``build_encoder_inputs``  -- system.cpp:62-95
* ``llm_to_rvq``            -- rvq.cpp:112-132 (safe mode raises on a level mismatch)
* ``roll_context``          -- system.cpp:320-333
* ``StreamingSession``      -- system.cpp:177-333 without the codec: per-chunk
  seed = base seed + chunk index (cli/main.cpp:459,599), encoder re-run on the
  sliding 10 s context, tokens decoded on the device, context kept on the host.
* ``DeviceStreamingSession`` -- the same with the context on the device
  (``mrt_df.Stream``): encoder inputs, llm_to_rvq and the roll run as HIP
  kernels, and ``pipeline_encoder`` enqueues the next chunk's encoder early
  (system.cpp:334-370).
"""

from __future__ import annotations

import dataclasses
from typing import Optional, Sequence

import numpy as np

import mrt_df


@dataclasses.dataclass(frozen=True)
class SystemConfig:
    """system.h:44-83 (values of the reference's SystemConfig)."""

    chunk_frames: int = 50
    context_frames: int = 250
    codebook_size: int = 1024
    encoder_codec_rvq_depth: int = 4
    encoder_style_rvq_depth: int = 6
    decoder_codec_rvq_depth: int = 16
    mask_token: int = 1
    codec_offset: int = 2

    @property
    def style_offset(self) -> int:
        return self.codec_offset + self.decoder_codec_rvq_depth * self.codebook_size + 1024

    @property
    def encoder_length(self) -> int:
        return self.context_frames * self.encoder_codec_rvq_depth + self.encoder_style_rvq_depth


def build_encoder_inputs(context: np.ndarray, cfg: SystemConfig,
                         style: Optional[Sequence[int]]) -> np.ndarray:
    """(context_frames, 16) RVQ ids (-1 = empty) + style ids -> (2, enc_len) int32."""
    ctx = np.asarray(context, dtype=np.int32)
    e, s = cfg.encoder_codec_rvq_depth, cfg.encoder_style_rvq_depth
    frames = ctx.shape[0]
    out = np.empty((2, frames * e + s), dtype=np.int32)
    lv = np.arange(e, dtype=np.int32)[None, :] * cfg.codebook_size
    v = ctx[:, :e]
    codec = np.where(v >= 0, cfg.codec_offset + lv + v, cfg.mask_token).reshape(-1)
    out[0, :frames * e] = codec
    out[1, :frames * e] = codec
    if style is None:
        out[0, frames * e:] = cfg.mask_token
    else:
        st = np.asarray(style, dtype=np.int32)
        if st.shape != (s,):
            raise ValueError("style_tokens_lm size != encoder_style_rvq_depth")
        out[0, frames * e:] = st
    out[1, frames * e:] = cfg.mask_token
    return out


def llm_to_rvq(tokens: np.ndarray, codebook_size: int, offset: int, safe: bool = True) -> np.ndarray:
    t = np.asarray(tokens, dtype=np.int32)
    shifted = t - offset
    r = np.mod(shifted, codebook_size)
    if safe:
        lv = np.arange(t.shape[-1], dtype=np.int32) * codebook_size
        if np.any((shifted - r) != lv):
            raise ValueError("llm_to_rvq: token levels do not match expected RVQ structure")
    return r.astype(np.int32)


def roll_context(context: np.ndarray, new_rvq: np.ndarray) -> np.ndarray:
    ctx = np.asarray(context, dtype=np.int32)
    n = new_rvq.shape[0]
    out = np.empty_like(ctx)
    out[:-n] = ctx[n:]
    out[-n:] = new_rvq
    return out


class StreamingSession:
    """Chunk-by-chunk token generation with a carried context (system.cpp:177-333)."""

    def __init__(self, model: "mrt_df.Depthformer", cfg: SystemConfig = SystemConfig(),
                 style: Optional[Sequence[int]] = None, seed: int = 0, temperature: float = 1.1,
                 top_k: int = 40, guidance_weight: float = 5.0, use_graph: bool = True):
        self.model, self.cfg, self.style = model, cfg, style
        self.state = model.new_state(rows=2, max_frames=cfg.chunk_frames, enc_len=cfg.encoder_length)
        self.context = np.full((cfg.context_frames, cfg.decoder_codec_rvq_depth), -1, dtype=np.int32)
        self.chunk_index = 0
        self.last_llm: Optional[np.ndarray] = None
        self.base_seed = seed
        self.opts = mrt_df.GenOptions(num_frames=cfg.chunk_frames, rvq_depth=cfg.decoder_codec_rvq_depth,
                                      temperature=temperature, top_k=top_k,
                                      guidance_weight=guidance_weight, codebook_size=cfg.codebook_size,
                                      codec_offset=cfg.codec_offset, use_graph=use_graph)

    def generate_chunk(self) -> np.ndarray:
        """Returns the chunk's (50, 16) RVQ ids and advances the context."""
        enc = build_encoder_inputs(self.context, self.cfg, self.style)
        self.opts.seed = self.base_seed + self.chunk_index
        llm = self.state.generate_tokens(enc, self.opts)
        self.last_llm = llm
        rvq = llm_to_rvq(llm, self.cfg.codebook_size, self.cfg.codec_offset)
        self.context = roll_context(self.context, rvq)
        self.chunk_index += 1
        return rvq


class DeviceStreamingSession:
    """StreamingSession with the RVQ context resident on the device."""

    def __init__(self, model: "mrt_df.Depthformer", cfg: SystemConfig = SystemConfig(),
                 style: Optional[Sequence[int]] = None, seed: int = 0, temperature: float = 1.1,
                 top_k: int = 40, guidance_weight: float = 5.0, use_graph: bool = True,
                 pipeline_encoder: bool = True):
        self.model, self.cfg, self.style = model, cfg, style
        self.stream = mrt_df.Stream(model, mrt_df.StreamConfig(
            chunk_frames=cfg.chunk_frames, context_frames=cfg.context_frames,
            codebook_size=cfg.codebook_size, encoder_codec_rvq_depth=cfg.encoder_codec_rvq_depth,
            encoder_style_rvq_depth=cfg.encoder_style_rvq_depth,
            decoder_codec_rvq_depth=cfg.decoder_codec_rvq_depth, mask_token=cfg.mask_token,
            codec_offset=cfg.codec_offset))
        self.state = self.stream.state
        self.base_seed = seed
        self.opts = mrt_df.ChunkOptions(temperature=temperature, top_k=top_k,
                                        guidance_weight=guidance_weight,
                                        pipeline_encoder=pipeline_encoder, use_graph=use_graph)
        self.last_llm: Optional[np.ndarray] = None
        self.last_audio: Optional[np.ndarray] = None
        self.codec = None

    def attach_codec(self, codec: "mrt_df.Codec") -> None:
        """From now on each chunk also returns audio (the whole generate_chunk)."""
        self.stream.attach_codec(codec)
        self.codec = codec

    @property
    def chunk_index(self) -> int:
        return self.stream.chunk_index

    @property
    def context(self) -> np.ndarray:
        return self.stream.get_context()[0]

    def generate_chunk(self) -> np.ndarray:
        """Returns the chunk's (50, 16) RVQ ids and advances the device context."""
        self.opts.seed = self.base_seed + self.chunk_index
        if self.codec is not None:
            self.last_llm, rvq, self.last_audio = self.stream.generate_chunk_audio(self.style, self.opts)
        else:
            self.last_llm, rvq = self.stream.generate_chunk(self.style, self.opts)
        return rvq
