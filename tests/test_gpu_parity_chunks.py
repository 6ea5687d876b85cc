"""bf16 parity of the benchmarked kernel -- the frame kernel, one launch per
frame -- over whole 2 s chunks (50 frames x 16 levels) at the benchmark dims
(d_model 1024, 16 heads x 64, d_ff 2816, 12/20/4 layers, vocab 29824, 1006
encoder tokens), through the C ABI.

The checker is the C restatement of the oracle (oracle/df_cpu.c, pinned to the
numpy oracle in tests/test_oracle_c.py), run in fp32 and in bf16-emulating
precision on the tokens the device fed, with the chunk criterion of
chunk_check.assert_bf16_chunk: every (frame, level) slice within 2e-2 of the
fp32 oracle, the chunk's RMS slice error within 1.25 x the bf16 oracle's own,
CFG argmax agreement with fp32 at least the bf16 oracle's less 0.05, and every
argmax flip a near-tie.

  * teacher-forced chunks for four (weight seed, token seed) pairs;
  * a free-running chunk (top-k 40, T 1.1, w 5, the streaming defaults): every
    draw is the oracle sampler's draw from the logits the device recorded for
    it (draw_check.assert_draws), and the oracle teacher-forced on the
    device's own tokens meets the criterion;
  * the free-running tokens of the speculative path (committed fixture,
    tests/golden/make_spec_tokens.py) through the plain frame kernel.
"""

from __future__ import annotations

import dataclasses
import os
import pathlib

import numpy as np
import pytest
from chunk_check import assert_bf16_chunk
from draw_check import assert_draws

pytestmark = pytest.mark.gpu

SEEDS = [(1234, 42), (7, 101), (99, 202), (2024, 303)]
GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "spec_free_running_tokens.npz"


@pytest.fixture(scope="module")
def mods(gpu_available):
    import mrt_df
    import synth_bundle
    import system
    from oracle import depthformer_oracle as O
    from oracle import df_cpu
    df_cpu.CpuDepthformer.set_threads(min(16, os.cpu_count() or 1))
    return dict(mrt_df=mrt_df, synth_bundle=synth_bundle, system=system, O=O, df_cpu=df_cpu,
                cfg=mrt_df.Config.bench())


def _enc_tokens(m, tseed):
    system = m["system"]
    scfg = system.SystemConfig()
    rng = np.random.default_rng(tseed)
    ctx = np.stack([rng.integers(0, 1024, scfg.context_frames) for _ in range(16)], axis=1).astype(np.int32)
    style = scfg.style_offset + 1024 * np.arange(6) + rng.integers(0, 1024, 6)
    return system.build_encoder_inputs(ctx, scfg, style), rng


def _device(m, w, tok, F, opts, teacher=None):
    import torch
    model = m["mrt_df"].Depthformer(w, m["cfg"], dtype="bf16")
    st = model.new_state(max_frames=F)
    rec = dict(slices=torch.zeros((F, 16, 2, 1024), dtype=torch.float32, device="cuda"),
               drawn=torch.zeros((F, 16), dtype=torch.int32, device="cuda"))
    toks = st.generate_tokens(tok, opts, teacher=teacher, record=rec)
    out = dict(tokens=toks, slices=rec["slices"].cpu().numpy(), drawn=rec["drawn"].cpu().numpy())
    st.close()
    model.close()
    return out


def _oracle_slices(m, w, tok, tokens, seed):
    """Level slices of the C oracle in fp32 and bf16, teacher-forced on `tokens`."""
    O, df_cpu = m["O"], m["df_cpu"]
    ocfg = O.DepthformerConfig(**dataclasses.asdict(m["cfg"]))
    F = tokens.shape[0]
    opts = O.GenerateOptions(num_frames=F, rvq_depth=16, temperature=1.1, top_k=40, guidance_weight=5.0, seed=seed,
                             codebook_size=1024, codec_offset=2)
    out = {}
    for mode in ("fp32", "bf16"):
        cm = df_cpu.CpuDepthformer(w, ocfg, max_frames=F, mode=mode)
        cm.set_cross_from_encoder(cm.encode(tok))
        rec = {}
        fed = cm.generate(opts, teacher=tokens, record=rec)
        np.testing.assert_array_equal(fed, tokens)
        out[mode] = rec["slices"]
        del cm
    return out


def _gen_opts(m, F, seed):
    return m["mrt_df"].GenOptions(num_frames=F, rvq_depth=16, temperature=1.1, top_k=40, guidance_weight=5.0,
                                  seed=seed, codebook_size=1024, codec_offset=2)


@pytest.mark.parametrize("wseed,tseed", SEEDS)
def test_bf16_teacher_forced_chunk(mods, wseed, tseed):
    m = mods
    w = m["synth_bundle"].make_weights(m["cfg"], seed=wseed, threads=16)
    tok, rng = _enc_tokens(m, tseed)
    F = 50
    teacher = (2 + 1024 * np.arange(16)[None, :] + rng.integers(0, 1024, (F, 16))).astype(np.int32)
    g = _device(m, w, tok, F, _gen_opts(m, F, 5), teacher=teacher)
    np.testing.assert_array_equal(g["tokens"], teacher)
    o = _oracle_slices(m, w, tok, teacher, 5)
    figs = assert_bf16_chunk(g["slices"], o["bf16"], o["fp32"])
    print(f"chunk seeds ({wseed}, {tseed}): {figs}", flush=True)


def test_bf16_free_running_chunk(mods):
    m = mods
    O = m["O"]
    w = m["synth_bundle"].make_weights(m["cfg"], seed=1234, threads=16)
    tok, _ = _enc_tokens(m, 42)
    F, seed = 50, 5
    g = _device(m, w, tok, F, _gen_opts(m, F, seed))
    np.testing.assert_array_equal(g["tokens"], g["drawn"])  # free running: the fed ids are the draws
    guided = np.array([[O.cfg_combine(g["slices"][f, l], 5.0) for l in range(16)] for f in range(F)])
    ties = assert_draws(O, g["drawn"], guided, temperature=1.1, top_k=40, seed=seed, offset=2, codebook=1024,
                        max_ties=8)
    lo = 2 + 1024 * np.arange(16)[None, :]
    assert ((g["tokens"] >= lo) & (g["tokens"] < lo + 1024)).all()
    o = _oracle_slices(m, w, tok, g["tokens"], seed)
    figs = assert_bf16_chunk(g["slices"], o["bf16"], o["fp32"])
    print(f"free-running chunk: {ties} ulp ties of 800 draws; {figs}", flush=True)


@pytest.mark.parametrize("which", ["drafted", "fixed_point"])
def test_bf16_speculative_path_tokens(mods, which):
    m = mods
    fx = np.load(GOLDEN)
    w = m["synth_bundle"].make_weights(m["cfg"], seed=1234, threads=16)
    tok, tokens = fx["enc_tokens"], fx[which].astype(np.int32)
    F = tokens.shape[0]
    g = _device(m, w, tok, F, _gen_opts(m, F, 4), teacher=tokens)
    o = _oracle_slices(m, w, tok, tokens, 4)
    # two frames (32 slices): the RMS ratio is taken over few slices, so its
    # bound is wider; the per-slice bound against fp32 is the same
    figs = assert_bf16_chunk(g["slices"], o["bf16"], o["fp32"], delta=0.5, slack=0.15)
    print(f"speculative-path tokens ({which}): {figs}", flush=True)
