#!/usr/bin/env python3
"""Bench: the MoE-64 bottleneck transformer (d256, 16 blocks, 64 experts, top-1,
68x120 tokens, Zipf(1.1) routing) on one MI355X.

One step = one pass of the whole 16-block chain over one batch of frames
(default 16 frames = 130,560 tokens), replayed from the engine's hipGraph.
Inputs and weights are resident in HBM before timing starts. Prints one JSON
line (see the keys below); everything else goes to stderr.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch 16]
"""
import argparse
import json
import os
import platform
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "prism-inference_amd"))

import prism_amd as P  # noqa: E402

MFMA_F16_PEAK = 2.5e15   # dense fp16 MFMA, MI355X
HBM_PEAK = 8.0e12        # HBM3E bytes/s, MI355X
METRIC = "frames/s + us/frame, MoE-64exp d256x16blk @68x120 tok; % fp16 MFMA peak"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def attn_flops_per_token(cfg):
    d = cfg.dim
    return 2 * (3 * d * d + 2 * 64 * d + d * d)


def router_flops_per_token(cfg):
    return 2 * cfg.dim * cfg.n_experts if cfg.n_experts > 1 else 0


def time_graph(hip, eng, dx, dy, batch, steps, warmup, stream, adapted=False):
    for _ in range(warmup):
        eng.forward(dx, dy, batch, stream, graph=True, adapted=adapted)
    hip.sync()
    e0, e1 = hip.event(), hip.event()
    t0 = time.perf_counter()
    hip.record(e0, stream)
    for _ in range(steps):
        eng.forward(dx, dy, batch, stream, graph=True, adapted=adapted)
    hip.record(e1, stream)
    ms = hip.elapsed_ms(e0, e1)
    hip.sync()
    wall = time.perf_counter() - t0
    return ms / steps, wall


def time_stage(hip, launch, reps, stream):
    """Average duration (ms) of one stage launch, HIP events on its stream."""
    for _ in range(3):
        rc = launch()
        assert rc == 0
    hip.sync()
    e0, e1 = hip.event(), hip.event()
    hip.record(e0, stream)
    for _ in range(reps):
        launch()
    hip.record(e1, stream)
    return hip.elapsed_ms(e0, e1) / reps


def time_e2e(hip, eng, frame, display, steps, warmup, stream):
    """ms per end-to-end frame (batch 1), hipGraph replay, HIP events on the stream."""
    for _ in range(warmup):
        eng.forward_e2e(frame, display, 1, stream, graph=True)
    hip.sync()
    e0, e1 = hip.event(), hip.event()
    hip.record(e0, stream)
    for _ in range(steps):
        eng.forward_e2e(frame, display, 1, stream, graph=True)
    hip.record(e1, stream)
    return hip.elapsed_ms(e0, e1) / steps


# Encoder / decoder stages: (name, input channels at its input resolution,
# skip channels, output channels, input res index, output res index, MACs per
# output pixel). dec1's output is the 12-channel render-resolution map that its
# kernel shuffles to the display (3 x 2x2 per pixel); its MACs include the
# 32 -> 12 output conv.
CODEC_STAGES = [("enc0", 9, 0, 32, 0, 0, 32 * 81), ("enc1", 32, 0, 64, 0, 1, 64 * 288),
                ("enc2", 64, 0, 128, 1, 2, 128 * 576), ("enc3", 128, 0, 128, 2, 3, 128 * 1152),
                ("dec3", 128, 128, 128, 3, 2, 128 * 256), ("dec2", 128, 64, 64, 2, 1, 64 * 192),
                ("dec1_out", 64, 32, 12, 1, 0, 32 * 96 + 12 * 32)]


def codec_section(hip, eng, desc, steps, warmup, reps, stream):
    """The end-to-end frame at batch 1 and each codec stage's duration, with
    its algorithmic HBM bytes (input map + skip map + output map + weights,
    each once) against the 8 TB/s peak."""
    cblob, coffs, _ = P.synth_codec(desc, seed=3)
    eng.load_codec(cblob, coffs)
    r = P.codec_resolutions()
    pix = [w * h for w, h in r]
    w0, h0 = r[0]
    frame, disp = hip.malloc(9 * pix[0] * 2), hip.malloc(12 * pix[0] * 2)
    hip.upload(frame, P.synth_normal(9 * pix[0], seed=4))
    ms_e2e = time_e2e(hip, eng, frame, disp, steps, warmup, stream)
    # per stage, on maps the encoder just wrote (so every input is realistic)
    bufs = {}
    for name, cin, cskip, cout, ri, ro, macs in CODEC_STAGES:
        bufs[name] = hip.malloc(pix[ro] * cout * 2)
    b3 = hip.malloc(pix[3] * 128 * 2)
    eng.encode(frame, b3, 1)
    hip.sync()
    src = {"enc0": (frame, None), "enc1": (bufs["enc0"], None), "enc2": (bufs["enc1"], None),
           "enc3": (bufs["enc2"], None), "dec3": (b3, bufs["enc2"]), "dec2": (bufs["dec3"], bufs["enc1"]),
           "dec1_out": (bufs["dec2"], bufs["enc0"])}
    stages = {}
    wbytes_all = 0
    for st, (name, cin, cskip, cout, ri, ro, macs) in enumerate(CODEC_STAGES):
        x, skip = src[name]
        y = bufs[name]
        ms = time_stage(hip, lambda: eng.L.prism_codec_stage(eng.h, st, x, skip, y, 1, stream), reps, stream)
        wbytes = macs * 2
        wbytes_all += wbytes
        nbytes = pix[ri] * cin * 2 + pix[ro] * (cskip + cout) * 2 + wbytes
        stages[name] = {"ms": round(ms, 5), "bytes": int(nbytes), "hbm_frac": round(nbytes / (ms * 1e-3) / HBM_PEAK, 4),
                        "tflops": round(2 * macs * pix[ro] / (ms * 1e-3) / 1e12, 2)}
    total = sum(v["ms"] for v in stages.values())
    # the frame's own codec launches: prism_encode (enc0 + enc1 in one launch,
    # enc1's taps read from the workgroup's e0 region in LDS; then enc2 + enc3
    # in one launch, enc3's taps read from the workgroup's e2 region) and
    # prism_decode (dec3, then dec2 + dec1 + output in one launch, the dec2 map
    # kept in LDS)
    t_enc = time_stage(hip, lambda: eng.L.prism_encode(eng.h, frame, b3, 1, stream), reps, stream)
    t_dec = time_stage(hip, lambda: eng.L.prism_decode(eng.h, b3, disp, 1, stream), reps, stream)
    for ptr in list(bufs.values()) + [frame, disp, b3]:
        hip.free(ptr)
    return {"frame_ms": round(ms_e2e, 5), "frames_per_s": round(1e3 / ms_e2e, 2),
            "codec_ms": round(total, 5),
            "codec_hbm_frac": round(sum(v["bytes"] for v in stages.values()) / (total * 1e-3) / HBM_PEAK, 4),
            "frame_codec_launches": {"encode_ms": round(t_enc, 5), "decode_ms": round(t_dec, 5),
                                     "note": "prism_encode (enc0 + enc1 in one launch, then enc2 + enc3 in one) and prism_decode "
                                             "(dec3, then dec2 + dec1 + output conv + PixelShuffle/sigmoid in one "
                                             "launch), back to back; codec_ms and stages are the seven stage calls"},
            "stages": stages,
            "workload": f"render {w0}x{h0} (9-channel frame) -> encoder -> proj 128->256 -> 16 MoE-64 blocks at "
                        f"{r[3][0]}x{r[3][1]} -> proj 256->128 -> decoder -> 3x{2 * w0}x{2 * h0} display, batch 1, "
                        "hipGraph replay; codec weights ~N(0, 2/K)"}


def chain_launches(eng, dx, dy, batch, stream, reps=5):
    """The chain's own attention and expert launches, run one after another
    (prism_chain_launch_times: the kernels, grids and arguments of
    prism_forward, HIP events between launches on the launch stream): median
    over `reps` chains of the mean launch durations (ms), and the grids."""
    a, e = [], []
    ga = ge = 0
    for _ in range(reps):
        ta, te, ga, ge = eng.chain_launch_times(dx, dy, batch, stream)
        a.append(ta)
        e.append(te)
    return statistics.median(a), statistics.median(e), ga, ge


def expert_kernel(d, tokens, n_experts):
    """The expert kernel the engine's chain launches for `tokens` tokens: 128-
    token tiles for d256 grids of >= 512 of them, else 64-token tiles (8 waves
    below 512); grids hold ceil(tokens / tile) + one partial tile per expert,
    rounded up to 8."""
    part = n_experts if n_experts > 1 else 0
    tiles = lambda bm: ((tokens + bm - 1) // bm + part + 7) // 8 * 8
    if d == 256 and tiles(128) >= 512:
        return f"prism_expert_d{d}_bm128"
    return f"prism_expert_d{d}_bm64" + ("_w8" if tiles(64) < 512 else "")


def measured_traffic(kernel, grid):
    """HBM bytes per dispatch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summaries (profiles/traffic_*_moe64_b16.txt, calibrated against a device
    copy of known size), if one covers this kernel at this grid; None
    otherwise."""
    pdir = os.path.join(ROOT, "profiles")
    if not os.path.isdir(pdir):
        return None, None
    for name in sorted(os.listdir(pdir)):
        if not (name.startswith("traffic_") and name.endswith("_moe64_b16.txt")):
            continue
        path = os.path.join(pdir, name)
        for line in open(path):
            if line.startswith("bench_traffic "):
                kv = dict(item.split("=", 1) for item in line.split()[1:])
                if kv.get("kernel") == kernel and int(kv.get("grid", -1)) == grid:
                    return int(kv["traffic_bytes"]), os.path.relpath(path, ROOT)
    return None, None


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(cfg, blob, offs, x_bits, budget_s, batch):
    """The oracle (fp32 C + OpenMP) on the host cores: batch-1 frames (median
    of up to 5 within the budget), then the whole batch once if the batch-1
    median says it fits the remaining budget."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    # OpenMP threads: the environment's OMP_NUM_THREADS if set (on a shared
    # GPU host, the CPU share that comes with one GPU), else every CPU this
    # process may run on; the host's own CPU count is reported beside it
    host_cpus = os.cpu_count() or 1
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else host_cpus
    env = os.environ.get("OMP_NUM_THREADS", "").strip()
    threads = int(env) if env.isdigit() and int(env) > 0 else usable
    threads_from = f"OMP_NUM_THREADS={env}" if env.isdigit() and int(env) > 0 else "all CPUs in the affinity mask"
    O.set_threads(threads)
    w = O.f16bits_to_f32(blob)
    n = cfg.H * cfg.W
    c1 = O.cfg(cfg.dim, cfg.n_heads, cfg.head_dim, cfg.n_experts, cfg.H, cfg.W, 1, True)
    x1 = O.f16bits_to_f32(x_bits[:n * cfg.dim]).reshape(n, cfg.dim)
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 and (time.perf_counter() - t_start) < budget_s:
        t0 = time.perf_counter()
        O.forward(c1, w, list(offs), x1)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    out = {"value": round(1.0 / med, 4), "unit": "frames/s", "cores": threads, "kind": "port",
           "cpu": cpu_model(), "omp_threads": O.max_threads(), "host_cpus": host_cpus, "affinity_cpus": usable,
           "threads_from": threads_from}
    sample = (f"{len(times)} frame(s) at batch 1 (8160 tokens x {cfg.n_blocks} blocks each), median "
              f"{med * 1e3:.1f} ms/frame")
    left = budget_s * 2 - (time.perf_counter() - t_start)
    if batch > 1 and med * batch < left:
        cb = O.cfg(cfg.dim, cfg.n_heads, cfg.head_dim, cfg.n_experts, cfg.H, cfg.W, batch, True)
        xb = O.f16bits_to_f32(x_bits[:batch * n * cfg.dim]).reshape(batch * n, cfg.dim)
        t0 = time.perf_counter()
        O.forward(cb, w, list(offs), xb)
        tb = time.perf_counter() - t0
        out["batch"] = {"frames": batch, "s": round(tb, 3), "frames_per_s": round(batch / tb, 4)}
        sample += f"; the batch of {batch} once, {tb:.2f} s"
    out["sample"] = sample + (f"; fp32 oracle (oracle/oracle.c) with OpenMP on {threads} threads ({threads_from}) "
                              f"of a host with {host_cpus} logical CPUs ({usable} in this process's affinity "
                              f"mask), host CPU: {cpu_model()}")
    return out


# The other workloads of the path, each at its stated batch and at batch 1
# (the headline MoE-64 line is the main measurement).
OTHER_CONFIGS = [("dense128", 16), ("std256", 16), ("moe16", 16), ("moe32", 4)]


def config_section(hip, name, batch, steps, stream):
    """ms per graph step at `batch` and at batch 1, and the chain's attention
    launch against the MFMA roofline, for one of the other workloads."""
    cfg = P.CONFIGS[name]
    desc = cfg.desc()
    blob, offs = P.synth_weights(desc, seed=0, routing=cfg.routing)
    eng = P.Engine(0)
    try:
        eng.load_weights(desc, blob, offs)
        T, d = cfg.tokens, cfg.dim
        dx, dy = hip.malloc(batch * T * d * 2), hip.malloc(batch * T * d * 2)
        try:
            hip.upload(dx, P.synth_features(cfg, batch=batch, seed=1))
            ms_b, _ = time_graph(hip, eng, dx, dy, batch, steps, 3, stream)
            ms_1, _ = time_graph(hip, eng, dx, dy, 1, steps, 3, stream)
            ta, te, ga, ge = chain_launches(eng, dx, dy, batch, stream, reps=3)
        finally:
            hip.free(dx)
            hip.free(dy)
    finally:
        eng.close()
    flops_frame = cfg.flops_per_token_block() * T * cfg.n_blocks
    S = max(1, min(2, batch // 2))  # the engine's sub-chains (CHAIN_SPLIT = 2 of >= 2 frames)
    tok_launch = batch * T // S
    a_flops = (attn_flops_per_token(cfg) + router_flops_per_token(cfg)) * tok_launch
    e_flops = 2 * 2 * d * d * tok_launch
    fused = ge == 0  # dense d128 blocks: the FFN runs inside the attention launch
    if fused:
        a_flops += e_flops
    kern = f"prism_attn_d{d}" + ("_w8" if ga < 512 else "") + (f"_r{(cfg.n_experts + 15) // 16}" if cfg.n_experts > 1 else "") + ("_ffn" if fused else "")
    return {"batch": batch, "ms_per_step": round(ms_b, 5), "frames_per_s": round(batch / (ms_b * 1e-3), 2),
            "mfma_frac": round(flops_frame * batch / (ms_b * 1e-3) / MFMA_F16_PEAK, 4),
            "batch1_us_per_frame": round(ms_1 * 1e3, 2),
            "batch1_mfma_frac": round(flops_frame / (ms_1 * 1e-3) / MFMA_F16_PEAK, 4),
            "roofline": {"kernel": kern, "grid": ga, "avg_launch_ms": round(ta, 5),
                         "frac": round(a_flops / (ta * 1e-3) / MFMA_F16_PEAK, 4),
                         "expert_grid": ge, "expert_avg_launch_ms": None if fused else round(te, 5),
                         "expert_frac": None if fused else round(e_flops / (te * 1e-3) / MFMA_F16_PEAK, 4)},
            "workload": f"d{d} x {cfg.n_blocks} blocks, {cfg.n_heads}x{cfg.head_dim} heads, "
                        + (f"{cfg.n_experts} experts top-1, " if cfg.n_experts > 1 else "dense FFN, ")
                        + f"{cfg.H}x{cfg.W} tokens"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--config", default="moe64")
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--stage-reps", type=int, default=20)
    ap.add_argument("--no-configs", action="store_true", help="skip the other workloads' section")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: the block chain runs on one GPU "
              "(frames and windows would shard across GPUs with no exchange). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    cfg = P.CONFIGS[args.config]
    B = args.batch
    hip = P.Hip()
    if hip.device_count() < 1:
        raise SystemExit("bench.py: no HIP device")

    log(f"[bench] synthesising {cfg.name}: {cfg.n_blocks} blocks, {cfg.n_experts} experts")
    desc = cfg.desc()
    blob, offs = P.synth_weights(desc, seed=0, routing=cfg.routing)
    eng = P.Engine(0)
    eng.load_weights(desc, blob, offs)
    T, d = cfg.tokens, cfg.dim
    x = P.synth_features(cfg, batch=B, seed=1)
    stream = hip.stream()
    dx, dy = hip.malloc(B * T * d * 2), hip.malloc(B * T * d * 2)
    hip.upload(dx, x)

    # ---- batch-B throughput (the step) and batch-1 latency, hipGraph replay
    log(f"[bench] batch {B}: warmup {args.warmup}, steps {args.steps}")
    ms_b, wall_b = time_graph(hip, eng, dx, dy, B, args.steps, args.warmup, stream)
    if cfg.n_experts > 1:
        assign_ptr, ntok = eng.forward_assignments()
        assign = hip.download(np.empty(cfg.n_blocks * ntok, np.int32), assign_ptr).reshape(cfg.n_blocks, ntok)
    log(f"[bench] batch 1 latency")
    ms_1, _ = time_graph(hip, eng, dx, dy, 1, max(args.steps, 50), args.warmup, stream)

    flops_frame = cfg.flops_per_token_block() * T * cfg.n_blocks
    fps_b = B / (ms_b * 1e-3)
    weight_bytes = blob.nbytes
    io_bytes_1 = 2 * T * d * 2

    # ---- per-stage kernel durations (batch B), HIP events on the launch stream
    n = B * T
    N = cfg.n_experts
    feats = hip.malloc(2 * n * d * 2)
    hip.copy(feats, dx, n * d * 2)
    aux_n = P.aux_elems(N, n)
    aux = hip.malloc(aux_n * 4)
    hip.memset(aux, 0, aux_n * 4)
    moe = N > 1
    a_push = eng.attn_push(0, 0, n * d)
    log("[bench] per-stage timing")
    t_attn = time_stage(hip, lambda: eng.attn(a_push, feats, B, stream), args.stage_reps, stream)
    attn_grid = ((cfg.W + 7) // 8) * ((cfg.H + 7) // 8) * B
    kname = f"prism_attn_d{d}" + ("_w8" if attn_grid < 512 else "")
    if moe:
        r_push = eng.router_push(0, T, n * d, 0, n, n + N)
        e_push = eng.expert_push(0, T, n * d, 0, 0, n, n + N)
        # the chain's MoE-block kernel: attention + routing in one launch (plus
        # the one-workgroup counter clear the stage call issues before it)
        rr_push = eng.router_push(0, T, n * d, 0, n, n + N)
        t_route = time_stage(hip, lambda: eng.attn_route(a_push, rr_push, feats, aux, B, stream), args.stage_reps,
                             stream)
        # the router launch clears its counts itself; the expert stage only reads them
        t_router = time_stage(hip, lambda: eng.router(r_push, feats, aux, B, stream), args.stage_reps, stream)
        t_expert = time_stage(hip, lambda: eng.experts(e_push, feats, aux, B, stream), args.stage_reps, stream)
        kname += f"_r{(N + 15) // 16}"
        timed = "prism_attn_route stage call: the routed attention kernel + its 1-workgroup count copy"
    else:
        # dense blocks: attention, then the FFN as the expert stage with one expert
        e_push = eng.expert_push(0, T, n * d, 0)
        t_route, t_router = t_attn, None
        t_expert = time_stage(hip, lambda: eng.experts(e_push, feats, None, B, stream), args.stage_reps, stream)
        timed = "prism_attn stage call: the attention kernel"
    route_flops = (attn_flops_per_token(cfg) + router_flops_per_token(cfg)) * n
    route_tflops = route_flops / (t_route * 1e-3) / 1e12
    traffic, traffic_src = measured_traffic(kname, attn_grid) if cfg.name == "moe64" else (None, None)

    # ---- the step's own launches: the chain's attention and expert kernels at
    # the grids the graph replays (batch 16: two sub-chains of 8 frames), run
    # one after another with HIP events between them
    log("[bench] chain launches")
    c_attn, c_exp, c_ga, c_ge = chain_launches(eng, dx, dy, B, stream)
    S = max(1, min(2, B // 2))  # sub-chains of the engine (CHAIN_SPLIT = 2 of >= 2 frames)
    tok_launch = n // S
    c_attn_flops = (attn_flops_per_token(cfg) + router_flops_per_token(cfg)) * tok_launch
    c_exp_flops = 2 * 2 * d * d * tok_launch
    c_fused = c_ge == 0  # dense d128 blocks: the FFN runs inside the attention launch
    if c_fused:
        c_attn_flops, c_exp_flops = c_attn_flops + c_exp_flops, 0
    c_kname = (f"prism_attn_d{d}" + ("_w8" if c_ga < 512 else "") + (f"_r{(N + 15) // 16}" if moe else "")
               + ("_ffn" if c_fused else ""))
    c_ename = None if c_fused else expert_kernel(d, tok_launch, N)
    c_traffic, c_traffic_src = measured_traffic(c_kname, c_ga) if cfg.name == "moe64" else (None, None)
    c_etraffic, _ = measured_traffic(c_ename, c_ge) if cfg.name == "moe64" else (None, None)

    # ---- projection adapters: the stage launches at batch B, and the adapted
    # chain (up -> blocks -> down, the projections fused into the first and
    # last launches) as one graph step
    ablob, aoffs = P.synth_adapters(desc, seed=0)
    eng.load_adapters(ablob, aoffs)
    I = aoffs.in_dim
    proj = hip.malloc(n * (I + d) * 2)
    hip.upload(proj, P.synth_normal(n * I, seed=2))
    up_push = eng.project_push(True, T, 0, n * I)
    dn_push = eng.project_push(False, T, n * I, 0)
    t_up = time_stage(hip, lambda: eng.project(True, up_push, proj, B, stream), args.stage_reps, stream)
    t_dn = time_stage(hip, lambda: eng.project(False, dn_push, proj, B, stream), args.stage_reps, stream)
    ax, ay = hip.malloc(n * I * 2), hip.malloc(n * I * 2)
    hip.copy(ax, proj, n * I * 2)
    ms_ad, _ = time_graph(hip, eng, ax, ay, B, max(5, args.steps // 2), 2, stream, adapted=True)
    proj_bytes = n * (I + d) * 2 + (I * d * 2 + (I + d) * 4)  # activations in + out, weights + biases once
    adapters = {"up_ms": round(t_up, 5), "down_ms": round(t_dn, 5),
                "up_hbm_frac": round(proj_bytes / (t_up * 1e-3) / HBM_PEAK, 4),
                "down_hbm_frac": round(proj_bytes / (t_dn * 1e-3) / HBM_PEAK, 4),
                "bytes_per_launch": proj_bytes,
                "adapted_chain_ms_per_step": round(ms_ad, 5),
                "note": "up_ms/down_ms: the pw_project 128->256 (+ReLU) and 256->128 stage launches at batch "
                        + str(B) + "; the adapted chain runs them fused into the first attention and the last "
                        "expert launch"}
    for ptr in (proj, ax, ay):
        hip.free(ptr)
    # the reference's end-to-end frame renders at 960x540, which encodes to the 68x120 grid
    e2e = None
    if P.codec_resolutions()[-1] == (cfg.W, cfg.H):
        log("[bench] end-to-end frame and codec stages")
        e2e = codec_section(hip, eng, desc, max(20, args.steps // 2), 5, args.stage_reps, stream)

    # ---- expert load actually produced (all blocks, batch B)
    expert_load = None
    if moe:
        share = np.array([np.bincount(a, minlength=N).max() / a.size for a in assign])
        hist0 = np.bincount(assign[0], minlength=N)
        expert_load = {"hottest_share_block0": round(float(hist0.max() / hist0.sum()), 4),
                       "hottest_share_mean": round(float(share.mean()), 4),
                       "coldest_share_block0": round(float(hist0.min() / hist0.sum()), 5)}
    routing = {P.ROUTE_RANDOM: "N(0,0.02) router bias", P.ROUTE_UNIFORM: "uniform-load router bias",
               P.ROUTE_ZIPF: "Zipf(1.1)-fitted router bias",
               P.ROUTE_ADVERSARIAL: "adversarial router bias (half the tokens to one expert)"}[cfg.routing]

    out = {
        "metric": METRIC,
        "value": round(fps_b, 3),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_b, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights"
                + (f", {routing})" if moe else ")"),
        "config": {"workload": f"{cfg.name}: d{d} x {cfg.n_blocks} blocks, {cfg.n_heads}x{cfg.head_dim} heads, "
                               f"8x8 windows, " + (f"{N} experts top-1, " if moe else "dense FFN, ")
                               + f"{cfg.H}x{cfg.W} tokens, batch {B}",
                   "batch": B, "tokens_per_frame": T, "blocks": cfg.n_blocks, "experts": N,
                   "parallelism": "single GPU"},
        "us_per_frame": round(ms_b * 1e3 / B, 3),
        "mfma_frac": round(flops_frame * B / (ms_b * 1e-3) / MFMA_F16_PEAK, 4),
        "batch1": {"frames_per_s": round(1e3 / ms_1, 2), "us_per_frame": round(ms_1 * 1e3, 2),
                   "mfma_frac": round(flops_frame / (ms_1 * 1e-3) / MFMA_F16_PEAK, 4),
                   "hbm_frac": round((weight_bytes + io_bytes_1) / (ms_1 * 1e-3) / HBM_PEAK, 4)},
        "stages_ms": {"attention_routed": round(t_route, 5) if moe else None, "experts": round(t_expert, 5),
                      "attention_stage": round(t_attn, 5),
                      "router_stage": round(t_router, 5) if moe else None, "batch": B},
        "roofline": {"kernel": c_kname, "grid": c_ga, "bound": "mfma",
                     "achieved": round(c_attn_flops / (c_attn * 1e-3) / 1e12, 2),
                     "peak": MFMA_F16_PEAK / 1e12, "unit": "TFLOP/s",
                     "frac": round(c_attn_flops / (c_attn * 1e-3) / MFMA_F16_PEAK, 4), "traffic": c_traffic,
                     "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated)",
                     "traffic_source": c_traffic_src,
                     "flops_per_launch": c_attn_flops, "avg_launch_ms": round(c_attn, 5),
                     "timed": f"the batch-{B} chain's own attention launches ({c_ga} workgroups, {tok_launch} tokens "
                              "each), run one after another by prism_chain_launch_times: HIP events between "
                              "launches on the launch stream, median over 5 chains of the mean over the chain's "
                              f"{cfg.n_blocks * S} launches",
                     "chain_launches": {
                         "attention": {"kernel": c_kname, "grid": c_ga, "flops": c_attn_flops,
                                       "avg_launch_ms": round(c_attn, 5),
                                       "frac": round(c_attn_flops / (c_attn * 1e-3) / MFMA_F16_PEAK, 4),
                                       "traffic": c_traffic},
                         "experts": None if c_fused else {
                                     "kernel": c_ename, "grid": c_ge, "flops": c_exp_flops,
                                     "avg_launch_ms": round(c_exp, 5),
                                     "frac": round(c_exp_flops / (c_exp * 1e-3) / MFMA_F16_PEAK, 4),
                                     "traffic": c_etraffic},
                         "both": {"flops": c_attn_flops + c_exp_flops, "ms": round(c_attn + c_exp, 5),
                                  "frac": round((c_attn_flops + c_exp_flops) / ((c_attn + c_exp) * 1e-3)
                                                / MFMA_F16_PEAK, 4),
                                  "note": "one block of one sub-chain, its two launches alone on the GPU; the "
                                          "graph overlaps one sub-chain's expert launch with the other's "
                                          "attention launch"}},
                     "stage_call": {"kernel": kname, "grid": attn_grid, "flops": route_flops,
                                    "avg_launch_ms": round(t_route, 5),
                                    "frac": round(route_tflops * 1e12 / MFMA_F16_PEAK, 4), "traffic": traffic,
                                    "timed": timed}},
        "expert_load": expert_load,
        "wall_s_timed": round(wall_b, 3),
        "adapters": adapters,
        "e2e_frame": e2e,
    }
    hip.free(feats)
    hip.free(aux)

    if cfg.name == "moe64" and not args.no_configs:
        out["configs"] = {}
        for name, b in OTHER_CONFIGS:
            log(f"[bench] config {name} batch {b}")
            out["configs"][name] = config_section(hip, name, b, 10, stream)

    if not args.no_cpu:
        log("[bench] CPU baseline (oracle)")
        out["cpu_baseline"] = cpu_baseline(cfg, blob, offs, x.reshape(-1), args.cpu_budget, B)
    else:
        out["cpu_baseline"] = None
    hip.free(dx)
    hip.free(dy)
    eng.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
