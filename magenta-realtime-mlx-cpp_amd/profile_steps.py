"""Profiling driver: back-to-back depth_step / temporal_step launches and one
decode of a 50-frame chunk (one frame-kernel launch per frame, no graph) at
the benchmark dims, plus a calibration copy of known size, for rocprofv3
counter runs (FETCH_SIZE / WRITE_SIZE per dispatch) and kernel traces.

    python magenta-realtime-mlx-cpp_amd/profile_steps.py [--reps N] [--copy-mib M]
    python magenta-realtime-mlx-cpp_amd/profile_steps.py --batched 32 [--frames F]

--batched N instead runs N independent streams together: one encode of
2N x 1006 rows and one decode of F frames through the replayed frame graph.

    python magenta-realtime-mlx-cpp_amd/profile_steps.py --codec 51 [--reps N]

--codec F instead runs N codec decodes of F frames (RVQ ids -> audio, fp32,
seeded synthetic codec weights) after 2 untimed ones.

    python magenta-realtime-mlx-cpp_amd/profile_steps.py --style [--reps N]

--style instead runs N MusicCoCa text embeddings (one 12-id prompt in 128
slots, fp32, seeded synthetic weights) after 3 untimed ones.

    python magenta-realtime-mlx-cpp_amd/profile_steps.py --encoder B [--reps N]

--encoder B instead runs N encoder prefills of B streams (2B x 1006 rows: the
12 layers and the cross K/V projection of the 20 temporal layers) after one
untimed one, for matrix-core counter runs.

    python magenta-realtime-mlx-cpp_amd/profile_steps.py --read-sweep

--read-sweep instead measures the device's read bandwidth (mrt_probe_read_bandwidth:
one warm pass, then repeated reads of one buffer) at buffer sizes from 16 MiB to
4 GiB, to locate where re-reads stop being served by the 256 MB last-level cache.

    python magenta-realtime-mlx-cpp_amd/profile_steps.py --handoff

--handoff instead measures the latency floor of the persistent kernels' phase
hand-offs: one word bounced between workgroup 0 and workgroups on other CUs
(mrt_probe_pingpong), and all-gathers of tagged words among 8..256 workgroups
(mrt_probe_handoff), the shape of one phase of the frame kernel at 256 / 1024,
also with the first poll of each round delayed.

    python magenta-realtime-mlx-cpp_amd/profile_steps.py --timeline

--timeline instead sets MRT_TRACE_PHASES, decodes a 50-frame chunk once untimed
and once traced, and prints workgroup 0's per-phase timeline of frame 1 (the
temporal step's first 14 layers and depth level 1), labelled by phase part, as
averages per layer (mrt_df_state_phase_trace).

The copy (torch's device copy of M MiB, M above the 256 MB last-level cache)
reads and writes exactly M MiB; its counter readings give the scale factor
between the counters and bytes.
"""

from __future__ import annotations

import argparse
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
if str(HERE) not in sys.path:
    sys.path.insert(0, str(HERE))


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=4, help="passes over the 16 depth levels")
    ap.add_argument("--copy-mib", type=int, default=1024, help="calibration copy size (above the 256 MB MALL)")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--batched", type=int, default=0, help="streams of a batched decode (0: single stream)")
    ap.add_argument("--frames", type=int, default=50, help="frames of the batched decode")
    ap.add_argument("--codec", type=int, default=0, help="frames of codec decodes (0: Depthformer steps)")
    ap.add_argument("--style", action="store_true", help="MusicCoCa text embeddings instead")
    ap.add_argument("--encoder", type=int, default=0, help="streams of encoder-only prefills (0: none)")
    ap.add_argument("--read-sweep", action="store_true", help="read bandwidth against buffer size instead")
    ap.add_argument("--handoff", action="store_true", help="hand-off latency probes instead")
    ap.add_argument("--timeline", action="store_true", help="per-phase timeline of one frame instead")
    a = ap.parse_args()
    if a.timeline:
        import os
        os.environ["MRT_TRACE_PHASES"] = "1"  # read when the state is created

    if a.handoff:
        import mrt_df
        for peer in (1, 2, 4, 7, 8, 16, 64, 255):
            us = mrt_df.pingpong_latency(peer, 2000)
            print(f"[profile] ping-pong workgroup 0 <-> {peer:3d}: one-way {us:.3f} us", flush=True)
        for g in (8, 32, 64, 128, 256):
            for words in (256, 1024):
                if words >= g and words // g <= 256:
                    us = mrt_df.handoff_latency(g, words, 2000)
                    print(f"[profile] all-gather {g:3d} workgroups x {words:4d} words: {us:.3f} us per round",
                          flush=True)
        for delay in (4, 8, 12, 16, 20, 24, 32):
            us = mrt_df.handoff_latency(256, 1024, 2000, delay)
            print(f"[profile] all-gather 256 workgroups x 1024 words, first poll after {delay:2d} x 64 clocks: "
                  f"{us:.3f} us per round", flush=True)
        return

    if a.read_sweep:
        import mrt_df
        for mib in (16, 32, 48, 64, 72, 80, 88, 96, 98, 104, 112, 128, 130, 160, 192, 224, 256, 384, 1024, 4096):
            passes = max(2, min(200, (8 << 10) // mib))  # about 8 GiB read per size
            gbs = mrt_df.read_bandwidth(mib << 20, passes)
            print(f"[profile] read {mib:5d} MiB x {passes:3d} passes: {gbs:8.1f} GB/s", flush=True)
        return

    import torch
    import mrt_df
    import synth_bundle
    import system

    if a.codec:
        shape = synth_bundle.CodecShape.reference()
        codec = mrt_df.Codec(synth_bundle.make_codec_weights(shape), max_frames=a.codec)
        tok = np.random.default_rng(3).integers(0, 1024, size=(a.codec, 16)).astype(np.int32)
        for _ in range(2):
            codec.decode(tok)
        ms = []
        for _ in range(a.reps):
            codec.decode(tok)
            ms.append(codec.decode_time())
        print(f"[profile] codec {a.codec} frames: {np.mean(ms):.3f} ms per decode over {a.reps}", flush=True)
        codec.close()
        return

    if a.style:
        ccfg = mrt_df.CocaConfig()
        sm = mrt_df.StyleModel(synth_bundle.make_coca_weights(ccfg), ccfg)
        ids = np.zeros(ccfg.max_text_len, np.int32)
        pad = np.ones(ccfg.max_text_len, np.float32)
        ids[0], pad[0] = 1, 0
        ids[1:13], pad[1:13] = np.random.default_rng(5).integers(2, ccfg.vocab_size, 12), 0
        for _ in range(3):
            sm.embed_text(ids, pad)
        ms = []
        for _ in range(a.reps):
            sm.embed_text(ids, pad)
            ms.append(sm.embed_time())
        print(f"[profile] style model: {np.mean(ms):.3f} ms per embed_text over {a.reps}", flush=True)
        sm.close()
        return

    cfg = mrt_df.Config.bench()
    model = mrt_df.Depthformer(synth_bundle.make_weights(cfg, seed=a.seed, threads=16), cfg, dtype="bf16")
    scfg = system.SystemConfig()
    if a.encoder:
        rng = np.random.default_rng(11)
        toks = []
        for _ in range(a.encoder):
            ctx = rng.integers(0, 1024, size=(scfg.context_frames, 16)).astype(np.int32)
            style = scfg.style_offset + 1024 * np.arange(6) + rng.integers(0, 1024, 6)
            toks.append(system.build_encoder_inputs(ctx, scfg, style))
        b = mrt_df.Batch(model, a.encoder, max_frames=1)
        enc = np.concatenate(toks, axis=0)
        b.encode(enc)
        torch.cuda.synchronize()
        for _ in range(a.reps):
            b.encode(enc)
        torch.cuda.synchronize()
        print(f"[profile] {a.reps} encoder prefills of {a.encoder} streams", flush=True)
        b.close()
        model.close()
        return
    if a.batched:
        rng = np.random.default_rng(7)
        toks = []
        for _ in range(a.batched):
            ctx = rng.integers(0, 1024, size=(scfg.context_frames, 16)).astype(np.int32)
            style = scfg.style_offset + 1024 * np.arange(6) + rng.integers(0, 1024, 6)
            toks.append(system.build_encoder_inputs(ctx, scfg, style))
        b = mrt_df.Batch(model, a.batched, max_frames=a.frames)
        opts = mrt_df.GenOptions(num_frames=a.frames, rvq_depth=cfg.rvq_depth, temperature=1.1, top_k=40,
                                 guidance_weight=5.0, use_graph=True)
        seeds = [a.seed + s for s in range(a.batched)]
        b.generate_tokens(np.concatenate(toks, axis=0), opts, seeds=seeds)
        print(f"[profile] batched {a.batched} streams, {a.frames} frames: decode {b.decode_time():.2f} ms", flush=True)
        b.close()
        model.close()
        return
    st = model.new_state(rows=2, max_frames=scfg.chunk_frames, enc_len=scfg.encoder_length)
    rng = np.random.default_rng(42)
    ctx = np.stack([rng.integers(0, 1024, scfg.context_frames) + 0 for _ in range(16)], axis=1)
    style = scfg.style_offset + 1024 * np.arange(6) + rng.integers(0, 1024, 6)
    st.encode(system.build_encoder_inputs(ctx, scfg, style))
    if a.timeline:
        opts = mrt_df.GenOptions(num_frames=scfg.chunk_frames, rvq_depth=cfg.rvq_depth, temperature=1.1, top_k=40,
                                 guidance_weight=5.0, seed=a.seed, use_graph=False)
        st.generate_tokens(None, opts)
        st.generate_tokens(None, opts)
        ms, launches = st.decode_time()
        trace, mhz = st.phase_trace()
        print(f"[profile] traced decode of {scfg.chunk_frames} frames: {ms:.2f} ms, {launches} launches", flush=True)
        print_timeline(trace, mhz, cfg)
        st.close()
        model.close()
        return

    n = a.copy_mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[profile] calibration copy: {a.copy_mib} MiB read + {a.copy_mib} MiB written", flush=True)

    g = torch.Generator(device="cpu").manual_seed(7)
    x = torch.randn(2, cfg.d_model, generator=g).to(device="cuda", dtype=torch.bfloat16)
    logits = torch.empty(2, 1024, dtype=torch.float32, device="cuda")
    out = torch.empty_like(x)
    for _ in range(a.reps):
        for l in range(cfg.rvq_depth):
            st.depth_step(x, l, level=l, out=logits, sync=False)
    st.sync()
    print(f"[profile] {a.reps * cfg.rvq_depth} depth_step launches", flush=True)
    for f in range(scfg.chunk_frames):
        st.temporal_step(x, f, out=out, sync=False)
    st.sync()
    print(f"[profile] {scfg.chunk_frames} temporal_step launches", flush=True)
    opts = mrt_df.GenOptions(num_frames=scfg.chunk_frames, rvq_depth=cfg.rvq_depth, temperature=1.1, top_k=40,
                             guidance_weight=5.0, seed=a.seed, use_graph=False)
    st.generate_tokens(None, opts)
    ms, launches = st.decode_time()
    print(f"[profile] decode of {scfg.chunk_frames} frames: {launches} persistent launches, {ms:.2f} ms", flush=True)
    st.close()
    model.close()


# Trace points of workgroup 0 = (head 0, part 0) per decoder layer, in order
# (persist_kernels.hip run_stack: three per activation load -- start, poll
# complete, norm and barrier done -- and one after each GEMV, head 0's
# attention and the cross-attention partial / combine).
_DEPTH_LAYER = ["QKV issue", "QKV poll", "QKV norm", "QKV GEMV", "attention",
                "O issue", "O poll", "O barrier", "O GEMV",
                "up issue", "up poll", "up norm", "up GEMV",
                "down issue", "down poll", "down barrier", "down GEMV"]
_TEMPORAL_LAYER = (_DEPTH_LAYER[:9] + ["cross-q issue", "cross-q poll", "cross-q norm", "cross-q GEMV",
                                       "cross partial", "cross combine",
                                       "cross-O issue", "cross-O poll", "cross-O barrier", "cross-O GEMV"]
                   + _DEPTH_LAYER[9:])
_TRACE_START, _TRACE_END, _TRACE_DONE = 509, 510, 511


def _layer_deltas(row, t0, labels, nlayers):
    """Per-layer deltas (us) between consecutive stamps; the first delta of a
    layer runs from the previous layer's last stamp (t0 for layer 0)."""
    n = len(labels)
    out = []
    prev = t0
    for li in range(nlayers):
        pts = row[li * n:(li + 1) * n]
        if len(pts) < n or (pts == 0).any():
            break
        d = np.diff(np.concatenate([[prev], pts]).astype(np.int64))
        out.append(d)
        prev = pts[-1]
    return np.array(out, dtype=np.float64), prev


def print_timeline(trace, mhz, cfg):
    to_us = 1.0 / mhz
    # temporal step of frame 1: 400 stamps cover the first 14 of its layers
    t = trace[0]
    tl, _ = _layer_deltas(t, t[_TRACE_START], _TEMPORAL_LAYER, 14)
    tot_t = (int(t[_TRACE_DONE]) - int(t[_TRACE_START])) * to_us
    print(f"[profile] temporal step of frame 1: {tot_t:.2f} us total; mean over its first {len(tl)} layers:", flush=True)
    for lab, v in zip(_TEMPORAL_LAYER, tl.mean(0) * to_us):
        print(f"[profile]   {lab:16s} {v:6.2f} us", flush=True)
    print(f"[profile]   {'layer':16s} {tl.sum(1).mean() * to_us:6.2f} us", flush=True)
    # depth level 1 of frame 1: 4 layers, then the head's activation load
    d = trace[1]
    dl, last = _layer_deltas(d, d[_TRACE_START], _DEPTH_LAYER, cfg.num_depth_layers)
    tot_d = (int(d[_TRACE_DONE]) - int(d[_TRACE_START])) * to_us
    print(f"[profile] depth level 1 of frame 1: {tot_d:.2f} us total; mean over its {len(dl)} layers:", flush=True)
    for lab, v in zip(_DEPTH_LAYER, dl.mean(0) * to_us):
        print(f"[profile]   {lab:16s} {v:6.2f} us", flush=True)
    print(f"[profile]   {'layer':16s} {dl.sum(1).mean() * to_us:6.2f} us", flush=True)
    k = cfg.num_depth_layers * len(_DEPTH_LAYER)
    h = d[k:k + 3].astype(np.int64)
    if (h > 0).all():
        print(f"[profile]   {'head issue':16s} {(h[0] - int(last)) * to_us:6.2f} us", flush=True)
        print(f"[profile]   {'head poll':16s} {(h[1] - h[0]) * to_us:6.2f} us", flush=True)
        print(f"[profile]   {'head norm':16s} {(h[2] - h[1]) * to_us:6.2f} us", flush=True)
        print(f"[profile]   {'head GEMV + logit gather':16s} {(int(d[_TRACE_END]) - h[2]) * to_us:6.2f} us", flush=True)
        print(f"[profile]   {'draw + publish':16s} {(int(d[_TRACE_DONE]) - int(d[_TRACE_END])) * to_us:6.2f} us",
              flush=True)
        # inside the draw (sample_block): stamps after the guided logits, the argmax, the count of
        # candidates above it, the radix-select fallback (if taken), the publish, and each radix pass
        names = ["scaled+noise", "argmax", "count", "fallback", "publish", "radix 1", "radix 2", "radix 3", "radix 4"]
        marks = [f"{nm} {(int(v) - int(d[_TRACE_END])) * to_us:.2f}" for nm, v in zip(names, d[490:499]) if v]
        print("[profile]   draw stamps (us after the logit gather): " + ", ".join(marks), flush=True)
    # phase-part totals per depth level
    groups = {"issue next weights": ["issue"], "poll (hand-off + weights)": ["poll"],
              "norm / barrier": ["norm", "barrier"], "GEMV + stores": ["GEMV"], "attention (head 0)": ["attention"]}
    for name, keys in groups.items():
        cols = [i for i, lab in enumerate(_DEPTH_LAYER) if any(lab.endswith(k) or lab == k for k in keys)]
        print(f"[profile] depth level, {name}: {dl[:, cols].sum(1).sum() * to_us:.2f} us", flush=True)


if __name__ == "__main__":
    main()
