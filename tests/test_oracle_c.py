"""The C/OpenMP restatement of the decode steps (oracle/df_cpu.c) against the
numpy oracle, fp32, at the tiny dims: two independent restatements of
model.cpp:322-659 written separately must agree to float32 rounding over
several temporal and depth steps with their caches (and the caches too),
at 1 thread and at several."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import depthformer_oracle as O
from oracle import df_cpu

import synth_bundle


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.fixture(scope="module")
def env():
    df_cpu.build()
    cfg = O.DepthformerConfig.tiny()
    w = synth_bundle.make_weights(cfg, seed=9, norm_jitter=0.2)
    return cfg, w


@pytest.mark.parametrize("threads", [1, 4])
def test_c_steps_equal_numpy_oracle(env, threads):
    cfg, w = env
    df_cpu.CpuDepthformer.set_threads(threads)
    om = O.OracleDepthformer(w, cfg, mode="fp32")
    cm = df_cpu.CpuDepthformer(w, cfg, max_frames=6)
    rng = np.random.default_rng(threads)
    enc_tokens = rng.integers(0, cfg.vocab_size, (2, cfg.max_encoder_length))
    enc = om.encode(enc_tokens)
    cm.set_cross(om.precompute_cross_kv(enc))
    tcache = om.empty_temporal_cache()
    for f in range(6):
        x = rng.standard_normal((2, 1, cfg.d_model)).astype(np.float32)
        exp = om.temporal_step(x, enc, tcache, f)
        got = cm.temporal_step(x, f)
        assert rel(got, exp[:, 0]) <= 1e-5, f
        dcache = om.empty_depth_cache()
        for l in range(cfg.rvq_depth):
            y = rng.standard_normal((2, 1, cfg.d_model)).astype(np.float32)
            full = om.depth_step(y, dcache, l)
            if l % 2:
                got = cm.depth_step(y, l)
                assert rel(got, full) <= 1e-5, (f, l)
            else:
                got = cm.depth_step(y, l, level=l, codebook=8, codec_offset=2)
                assert rel(got, full[:, 2 + 8 * l: 2 + 8 * (l + 1)]) <= 1e-5, (f, l)
        for i in range(cfg.num_depth_layers):
            assert rel(cm.dk[i], dcache[i]["k"]) <= 1e-5
            assert rel(cm.dv[i], dcache[i]["v"]) <= 1e-5
    for i in range(cfg.num_temporal_layers):
        assert rel(cm.tk[i], tcache[i]["k"]) <= 1e-5
        assert rel(cm.tv[i], tcache[i]["v"]) <= 1e-5
