"""Writes tests/golden/spec_free_running_tokens.npz: the free-running tokens of
the speculative depth decoding run at the benchmark dims (bf16, d_model 1024,
16 heads x 64, d_ff 2816, 12/20/4 layers, weights seed 1234, encoder context
and style from seed 42; 2 frames, top-k 40, T 1.1, CFG w 5).  `drafted` are
the tokens of the first speculative call (seed 4, drafts = a seed-3 decode),
`fixed_point` those of the call that repeats itself (every draft accepted).
On these tokens the plain frame kernel, teacher-forced, was once measured
2.08e-2 from the bf16 oracle (1.72e-2 from fp32); the chunk-parity tests feed
them to the frame kernel as a fixed input.

    python tests/golden/make_spec_tokens.py      (needs the GPU)
"""

from __future__ import annotations

import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
for p in (ROOT, ROOT / "magenta-realtime-mlx-cpp_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

import mrt_df  # noqa: E402
import synth_bundle  # noqa: E402
import system  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent / "spec_free_running_tokens.npz"


def main() -> None:
    cfg = mrt_df.Config.bench()
    w = synth_bundle.make_weights(cfg, seed=1234, threads=16)
    model = mrt_df.Depthformer(w, cfg, dtype="bf16")
    scfg = system.SystemConfig()
    rng = np.random.default_rng(42)
    ctx = rng.integers(0, 1024, size=(scfg.context_frames, 16)).astype(np.int32)
    style = scfg.style_offset + 1024 * np.arange(6) + rng.integers(0, 1024, 6)
    tok = system.build_encoder_inputs(ctx, scfg, style)
    F, L = 2, 16
    st = model.new_state(max_frames=F)
    mk = lambda seed: mrt_df.GenOptions(num_frames=F, rvq_depth=L, temperature=1.1, top_k=40, guidance_weight=5.0,
                                        seed=seed, codebook_size=1024, codec_offset=2, speculative=True)
    st.generate_tokens(tok, mk(3))
    drafted = st.generate_tokens(None, mk(4))
    prev = drafted
    for _ in range(2 * (L + 2)):
        toks = st.generate_tokens(None, mk(4))
        if (toks == prev).all():
            break
        prev = toks
    else:
        raise RuntimeError("no fixed point")
    st.close()
    model.close()
    np.savez(OUT, enc_tokens=tok, drafted=drafted, fixed_point=toks)
    print(f"wrote {OUT}: drafted {drafted.tolist()}\nfixed point {toks.tolist()}")


if __name__ == "__main__":
    main()
