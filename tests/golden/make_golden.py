"""Writes tests/golden/tiny_decode.npz: oracle outputs of the tiny config
(d_model 128, 2 heads x 64, 2+2+2 layers, 16 levels of 8 codes) for seeded
weights and tokens.  The reference ships no golden vectors for this path
(its parity tests were not published), so these fixtures pin the oracle
against regressions and give the HIP tests a fixed target.

    python tests/golden/make_golden.py

Weights come from synth_bundle.make_weights(seed=1234, norm_jitter=0.1),
which derives every tensor from its own seed; the fixture stores a checksum
of each tensor so a change of the generator is detected.
"""

from __future__ import annotations

import dataclasses
import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
for p in (ROOT, ROOT / "magenta-realtime-mlx-cpp_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

from oracle import depthformer_oracle as O  # noqa: E402

import synth_bundle  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent / "tiny_decode.npz"
SEED, JITTER, C, F = 1234, 0.1, 8, 3


def inputs():
    cfg = O.DepthformerConfig.tiny()
    w = synth_bundle.make_weights(cfg, seed=SEED, norm_jitter=JITTER)
    rng = np.random.default_rng(42)
    S = cfg.max_encoder_length
    tok = np.zeros((2, S), dtype=np.int32)
    lvl = np.arange(S - 6) % 4
    tok[0, :S - 6] = 2 + C * lvl + rng.integers(0, C, S - 6)
    tok[1, :S - 6] = tok[0, :S - 6]
    tok[0, S - 6:] = 2 + 16 * C + C * np.arange(6) + rng.integers(0, C, 6)
    tok[1, S - 6:] = 1
    teacher = (2 + C * np.arange(16)[None, :] + rng.integers(0, C, (F, 16))).astype(np.int32)
    return cfg, w, tok, teacher


def options(seed=77):
    return O.GenerateOptions(num_frames=F, rvq_depth=16, temperature=1.1, top_k=4, guidance_weight=5.0,
                             seed=seed, codebook_size=C, codec_offset=2)


def checksums(w):
    return np.array([float(np.asarray(w[k], dtype=np.float64).sum()) for k in sorted(w)])


def compute():
    cfg, w, tok, teacher = inputs()
    out = dict(enc_tokens=tok, teacher=teacher, weight_checksums=checksums(w))
    for mode in ("fp32", "bf16"):
        om = O.OracleDepthformer(w, cfg, mode=mode)
        rec = {}
        O.generate_tokens(om, tok, options(), teacher=teacher, record=rec)
        for k in ("enc_out", "temporal_out", "slices", "frame_mean", "drawn"):
            out[f"{mode}_tf_{k}"] = np.asarray(rec[k], dtype=np.float32 if k != "drawn" else np.int32)
    om = O.OracleDepthformer(w, cfg, mode="fp32")
    rec = {}
    out["fp32_free_tokens"] = O.generate_tokens(om, tok, options(seed=2024), record=rec)
    out["fp32_free_drawn"] = rec["drawn"]
    return out


def main():
    np.savez_compressed(OUT, **compute())
    print(OUT, OUT.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
