"""MusicCoCa text path and style tokens on the GPU (style_model.cpp:76-121)
against the oracle, through the C ABI: every text layer's output and the
pooled embedding within 1e-4 (norm-wise relative, fp32 as the reference's
StyleModel), RVQ tokens of a given vector equal to the oracle's
rvq_quantization (rvq.cpp:24-62) exactly (the argmin margins are checked to be
far above fp32 rounding first), and the style ids equal offset + level *
codebook + token.  Tiny and the reference's dims, seeded synthetic weights."""

from __future__ import annotations

import numpy as np
import pytest

import synth_bundle
from oracle import musiccoca_oracle as M

pytestmark = pytest.mark.gpu

TOL = 1e-4


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _margins(vec, cb):
    """Per level, the gap between the two smallest distances (fp64)."""
    r = vec.astype(np.float64)
    gaps = []
    for k in range(cb.shape[0]):
        d = ((r[None, :] - cb[k].astype(np.float64)) ** 2).sum(-1)
        s = np.sort(d)
        gaps.append(s[1] - s[0])
        r = r - cb[k][np.argmin(d)]
    return np.array(gaps)


def _check(sm, cfg, w, prompts):
    import mrt_df
    oc = M.OracleCoca(w, M.CocaConfig(**{f: getattr(cfg, f) for f in vars(M.CocaConfig())}), "fp32")
    for raw in prompts:
        ids, pad = M.text_ids(raw, cfg.max_text_len)
        print(f"prompt of {len(raw)} ids, d_model {cfg.d_model}", flush=True)
        emb = sm.embed_text(ids, pad)
        rec = {}
        ref = oc.embed_text(ids, pad, rec)
        errs = {f"layer{i}": rel(sm.read(1 + i, (cfg.max_text_len, cfg.d_model)), rec[f"layer{i}"])
                for i in range(cfg.num_layers)}
        errs["embedding"] = rel(emb, ref)
        print({k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
        for k, v in errs.items():
            assert v <= TOL, (k, v)
        np.testing.assert_array_equal(sm.read(mrt_df.COCA_BUF_EMBEDDING, (cfg.d_model,)), emb)
        # the RVQ of the device embedding, on the device and in the oracle: the
        # same vector, so the tokens agree unless a level's two best distances
        # lie within fp32 rounding of each other (~sqrt(d) * eps * |r|^2)
        cb = w["codebooks"][:cfg.rvq_depth]
        gaps = _margins(emb, cb)
        near = 1e-5 * max(1.0, float((emb.astype(np.float64) ** 2).sum()))
        print(f"smallest argmin gap {gaps.min():.3g} (near-tie bound {near:.3g})", flush=True)
        tok = sm.tokenize()
        want = M.rvq_quantization(emb[None], cb)[0][0]
        if not np.array_equal(tok, want):
            k = int(np.argmax(tok != want))
            assert gaps[k] < near, (k, tok, want, gaps)
        np.testing.assert_array_equal(sm.tokenize(emb), tok)
        st = sm.style_tokens_lm(ids, 6, cfg.codebook_size, 17410, padding=pad)
        np.testing.assert_array_equal(st, 17410 + cfg.codebook_size * np.arange(6) + tok[:6])


def test_musiccoca_tiny(gpu_available):
    import mrt_df
    cfg = mrt_df.CocaConfig.tiny()
    w = synth_bundle.make_coca_weights(cfg)
    sm = mrt_df.StyleModel(w, cfg)
    rng = np.random.default_rng(0)
    _check(sm, cfg, w, [list(rng.integers(2, cfg.vocab_size, 7)), list(rng.integers(2, cfg.vocab_size, 40)), []])
    ids, pad = M.text_ids([5, 6], cfg.max_text_len)
    ids[3] = cfg.vocab_size
    with pytest.raises(mrt_df.MrtError):
        sm.embed_text(ids, pad)
    sm.close()


def test_musiccoca_full_size(gpu_available):
    import mrt_df
    cfg = mrt_df.CocaConfig()
    w = synth_bundle.make_coca_weights(cfg)
    sm = mrt_df.StyleModel(w, cfg)
    rng = np.random.default_rng(1)
    _check(sm, cfg, w, [list(rng.integers(2, cfg.vocab_size, 12))])
    assert sm.embed_time() > 0
    sm.close()


@pytest.mark.parametrize("size", ["tiny", "full"])
def test_musiccoca_graph_replays_match_eager(gpu_available, size):
    """The first embed_text enqueues its kernels directly, the second captures
    them into a HIP graph and later calls replay it: every replay, with eager
    work (RVQ tokenisation) and host synchronisation between them, gives
    bit-identical embeddings to the direct launches of a second model."""
    import mrt_df
    cfg = mrt_df.CocaConfig.tiny() if size == "tiny" else mrt_df.CocaConfig()
    w = synth_bundle.make_coca_weights(cfg)
    rng = np.random.default_rng(3)
    prompts = [M.text_ids(list(rng.integers(2, cfg.vocab_size, n)), cfg.max_text_len) for n in (9, 30)]
    sm = mrt_df.StyleModel(w, cfg)
    eager = []
    for ids, pad in prompts:  # one direct call per model: the eager results
        ref = mrt_df.StyleModel(w, cfg)
        eager.append(ref.embed_text(ids, pad))
        ref.close()
    first = sm.embed_text(*prompts[0])  # direct
    np.testing.assert_array_equal(first, eager[0])
    for rep in range(4):  # capture on the first of these, replays after
        i = (rep + 1) % 2
        print(f"{size}: call {rep + 2}, prompt {i}", flush=True)
        got = sm.embed_text(*prompts[i])
        np.testing.assert_array_equal(got, eager[i])
        sm.tokenize()
    sm.close()
