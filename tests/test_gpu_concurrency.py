"""Two states of one model driven from two host threads at the benchmark dims.

Each state's persistent kernels take one workgroup per CU (256 on MI355X) and
poll words that the rest of their own grid writes, so two grids must never
share the device.  The library orders every persistent unit of work (a decode
or a step launch) on one device through a device-wide gate, whatever threads
and streams enqueue it.  Checks: tokens of concurrent decodes (graph replay on
one thread, eager launches on the other, and the step entry points on a third
state) equal the sequential decodes bit for bit, and no poll times out.
"""

from __future__ import annotations

import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_two_states_on_two_threads_match_sequential(gpu_available):
    import torch

    import mrt_df
    import synth_bundle
    import system

    cfg = mrt_df.Config.bench()
    w = synth_bundle.make_weights(cfg, seed=1234, threads=16)
    model = mrt_df.Depthformer(w, cfg, dtype="bf16")
    scfg = system.SystemConfig()
    rng = np.random.default_rng(77)
    toks = []
    for _ in range(2):
        ctx = rng.integers(0, 1024, size=(scfg.context_frames, 16)).astype(np.int32)
        style = scfg.style_offset + 1024 * np.arange(6) + rng.integers(0, 1024, 6)
        toks.append(system.build_encoder_inputs(ctx, scfg, style))
    F = 4
    opts = [mrt_df.GenOptions(num_frames=F, rvq_depth=16, temperature=1.1, top_k=40, guidance_weight=5.0, seed=s,
                              codebook_size=1024, codec_offset=2, use_graph=g)
            for s, g in ((11, True), (22, False))]
    states = [model.new_state(max_frames=F) for _ in range(2)]
    seq = [states[i].generate_tokens(toks[i], opts[i]) for i in range(2)]
    # a third state runs step entry points concurrently (temporal + depth)
    st3 = model.new_state(max_frames=F)
    st3.encode(toks[0])
    x = torch.zeros((2, cfg.d_model), dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()
    ref_t = st3.temporal_step(x, 0).float().cpu().numpy()

    results, errors = {}, []

    def decode(i):
        try:
            for r in range(3):
                results[(i, r)] = states[i].generate_tokens(toks[i] if r == 0 else None, opts[i])
        except Exception as e:  # noqa: BLE001
            errors.append((i, repr(e)))

    def steps():
        try:
            for r in range(4):
                results[("t", r)] = st3.temporal_step(x, 0).float().cpu().numpy()
        except Exception as e:  # noqa: BLE001
            errors.append(("t", repr(e)))

    th = [threading.Thread(target=decode, args=(i,)) for i in range(2)] + [threading.Thread(target=steps)]
    for t in th:
        t.start()
    for t in th:
        t.join(timeout=300)
    assert not any(t.is_alive() for t in th), "a decode thread did not finish"
    assert not errors, errors
    for i in range(2):
        for r in range(3):
            np.testing.assert_array_equal(results[(i, r)], seq[i], err_msg=f"state {i} round {r}")
    for r in range(4):
        np.testing.assert_array_equal(results[("t", r)], ref_t)
    for st in states + [st3]:
        st.close()
    model.close()
