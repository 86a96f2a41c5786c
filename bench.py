"""Quantized-linear benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME] [--graph | --no-graph]

A step is one quantized matmul (qmm_quantized_matmul through the C ABI) over
one batch of synthetic input resident in HBM.  The default workload is the
nvfp4 fused gate+up decode GEMV (M=1, N=34816, K=5120): the metric is achieved
HBM GB/s over the algorithmic bytes (every weight, scale, input and output
byte counted once).  Timed calls rotate over distinct weight copies totalling
at least 512 MiB so each call reads weights from HBM, not the 256 MB
Infinity Cache.  The K timed calls are eager launches on one stream, as the
reference's engine makes them, queued behind a GPU sleep: the host enqueues all K
while the GPU sleeps, so the HIP events on the stream around them time K kernels
back to back and none of the host's launch work (checked on every timing: when the
host's enqueueing outlasts the sleep, the result is discarded and the calls are
timed as one HIP graph replay instead, queued behind an untimed replay).  Before
timing, batches of K launches run untimed for at least 1 s and 2000 launches (the
clocks ramp over the first few hundred launches); the figure is the median of five
timings.  --graph times the graph replay only, --no-graph unqueued eager launches.

With no --config, every workload the headline metric is quoted on is timed in
turn (HEADLINE_SET: the gate+up GEMV first, whose figures are the line's
`value`; the mxfp8 GEMV, the down projection at M = 1-3, the mxfp8 prefill
GEMM, the lm_head GEMV and the lm_head prefill GEMM), each reported under
`configs` with its own roofline and CPU baseline.

Prints ONE JSON line on stdout.  The CPU baseline is the oracle's
fp32-accumulating restatement, timed on the host on a bounded sample on every
thread of the job's CPU share.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT, ROOT / "oracle", ROOT / "mlx-runner_amd"):
    sys.path.insert(0, str(p))

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"fp8": 5000.0, "bf16": 2500.0}

CONFIGS = {
    "mxfp8_gemv": dict(mode="mxfp8", M=1, N=5120, K=5120, xscale=1.0,
                       workload="mxfp8 GEMV, x bf16 [1,5120], W [5120,5120]"),
    "gateup": dict(mode="nvfp4", M=1, N=34816, K=5120, xscale=1.0,
                   workload="nvfp4 fused gate+up decode GEMV, x bf16 [1,5120], W [34816,5120]"),
    "down_m1": dict(mode="nvfp4", M=1, N=5120, K=17408, xscale=0.5,
                    workload="nvfp4 down-proj skinny GEMM, x bf16 [1,17408], W [5120,17408]"),
    "down_m2": dict(mode="nvfp4", M=2, N=5120, K=17408, xscale=0.5,
                    workload="nvfp4 down-proj skinny GEMM, x bf16 [2,17408], W [5120,17408]"),
    "down_m3": dict(mode="nvfp4", M=3, N=5120, K=17408, xscale=0.5,
                    workload="nvfp4 down-proj skinny GEMM, x bf16 [3,17408], W [5120,17408]"),
    "prefill": dict(mode="mxfp8", M=4096, N=17408, K=5120, xscale=1.0,
                    workload="mxfp8 prefill GEMM, x bf16 [4096,5120], W [17408,5120]"),
    "lmhead": dict(mode="nvfp4", M=1, N=248320, K=5120, xscale=1.0,
                   workload="nvfp4 lm_head decode GEMV, x bf16 [1,5120], W [248320,5120]"),
    "lmhead_prefill": dict(mode="nvfp4", M=2048, N=248320, K=5120, xscale=1.0,
                           workload="nvfp4 lm_head prefill GEMM, x bf16 [2048,5120], W [248320,5120]"),
    # short prefill chunks (the last partial chunk, the tokens left after a prefix-cache hit,
    # src/engine.zig:364-382) on the gate / up projection shape
    **{f"prefill_m{M}_{mode}": dict(mode=mode, M=M, N=17408, K=5120, xscale=1.0,
                                    workload=f"{mode} short prefill GEMM, x bf16 [{M},5120], W [17408,5120]")
       for M in (16, 64, 256) for mode in ("mxfp8", "nvfp4")},
    "mlp_gateup_silu": dict(mode="nvfp4", M=1, N=17408, K=5120, xscale=1.0, mlp=True,
                            workload="nvfp4 MLP gate+up+SiLU*mul fused decode GEMV, x bf16 [1,5120], "
                                     "W_gate, W_up [17408,5120]"),
    "mlp_gateup_silu_m3": dict(mode="nvfp4", M=3, N=17408, K=5120, xscale=1.0, mlp=True,
                               workload="nvfp4 MLP gate+up+SiLU*mul fused MTP-verify skinny GEMM, x bf16 [3,5120], "
                                        "W_gate, W_up [17408,5120]"),
    "gateup_m3": dict(mode="nvfp4", M=3, N=34816, K=5120, xscale=1.0,
                      workload="nvfp4 gate+up MTP-verify skinny GEMM, x bf16 [3,5120], W [34816,5120]"),
    "dense_lmhead": dict(mode="bf16", M=1, N=248320, K=5120, xscale=1.0,
                         workload="dense bf16 lm_head decode GEMV (mxfp8 checkpoints), x bf16 [1,5120], "
                                  "W bf16 [248320,5120]"),
    "gdn_decode": dict(gdn=True, B=1, T=1, Hk=16, Hv=48, Dk=128, Dv=128,
                       workload="GDN recurrence decode step (src/gdn_packed.metal): B=1, T=1, Hk=16, Hv=48, "
                                "Dk=Dv=128, bf16 q/k/v/beta, f32 g and state [1,48,128,128]"),
    "gdn_prefill": dict(gdn=True, B=1, T=2048, Hk=16, Hv=48, Dk=128, Dv=128,
                        workload="GDN recurrence over a 2048-token prefill chunk: B=1, T=2048, Hk=16, Hv=48, "
                                 "Dk=Dv=128, bf16 q/k/v/beta, f32 g and state"),
}
DEFAULT = "gateup"

# Every quantized linear of one decoded token at the model's default sizes
# (H=5120, I=17408, V=248320; src/model.zig:40-59): (weight, N, K, calls per
# token, call site).  48 GDN layers and 16 full-attention layers.
CENSUS = [
    ("self_attn.q_proj", 12288, 5120, 16, "src/model.zig:929"),
    ("self_attn.k_proj", 1024, 5120, 16, "src/model.zig:940"),
    ("self_attn.v_proj", 1024, 5120, 16, "src/model.zig:944"),
    ("self_attn.o_proj", 5120, 6144, 16, "src/model.zig:979"),
    ("linear_attn.in_proj_qkv", 10240, 5120, 48, "src/model.zig:1066"),
    ("linear_attn.in_proj_z", 6144, 5120, 48, "src/model.zig:1068"),
    ("linear_attn.in_proj_b", 48, 5120, 48, "src/model.zig:1072"),
    ("linear_attn.in_proj_a", 48, 5120, 48, "src/model.zig:1074"),
    ("linear_attn.out_proj", 5120, 6144, 48, "src/model.zig:1230"),
    ("mlp.gate_proj", 17408, 5120, 64, "src/model.zig:906"),
    ("mlp.up_proj", 17408, 5120, 64, "src/model.zig:908"),
    ("mlp.down_proj", 5120, 17408, 64, "src/model.zig:914"),
    ("lm_head", 248320, 5120, 1, "src/model.zig:1309"),
    ("mtp.fc", 5120, 10240, 0, "src/mtp.zig:158"),  # MTP drafting only: not in the per-token sum
]
# Projections of one x that a grouped call runs as one matrix (the loader places them back to back).
CENSUS_GROUPS = {
    "linear_attn.in_proj_qkv+z+b+a (grouped)": ("linear_attn.in_proj_qkv", "linear_attn.in_proj_z",
                                                "linear_attn.in_proj_b", "linear_attn.in_proj_a"),
    "self_attn.q+k+v_proj (grouped)": ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"),
}
BITS = {"mxfp8": 8, "nvfp4": 4, "bf16": 16}
GROUP = {"mxfp8": 32, "nvfp4": 16, "bf16": None}
ROTATE_BYTES = 512 << 20


def algorithmic(cfg):
    M, N, K, mode = cfg["M"], cfg["N"], cfg["K"], cfg["mode"]
    mats = 2 if cfg.get("mlp") else 1  # the fused MLP reads a gate and an up matrix
    wbytes = mats * N * K * BITS[mode] // 8
    sbytes = mats * N * K // GROUP[mode] if GROUP[mode] else 0
    return dict(w=wbytes, s=sbytes, bytes=wbytes + sbytes + M * K * 2 + M * N * 2, flops=2 * mats * M * N * K)


def roofline_of(cfg, alg, sec_per_call):
    peak_mm = MFMA_PEAK_TFLOPS["fp8" if cfg["mode"] == "mxfp8" else "bf16"]
    if cfg["M"] <= 8 or alg["bytes"] / (HBM_PEAK_GBS * 1e9) >= alg["flops"] / (peak_mm * 1e12):
        achieved = alg["bytes"] / sec_per_call / 1e9
        return dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(achieved / HBM_PEAK_GBS, 4))
    achieved = alg["flops"] / sec_per_call / 1e12
    peak = MFMA_PEAK_TFLOPS["fp8" if cfg["mode"] == "mxfp8" else "bf16"]
    # The same achieved rate against the other dense peaks that bear on it: mxfp8 runs x as
    # exact E4M3 hi + lo, two fp8 MFMAs per product (its ceiling is half the fp8 peak);
    # nvfp4 runs the bf16 MFMA (E2M1 x E4M3 weights have up to 6 significant bits), set
    # beside the fp8 and MXFP4 peaks its format would have on a narrower MFMA.
    others = {"mxfp8": {"fp8_hilo_ceiling": 2500.0},
              "nvfp4": {"fp8_dense": 5000.0, "mxfp4_dense": 10100.0}}[cfg["mode"]]
    return dict(bound="mfma", achieved=round(achieved, 1), peak=peak, unit="TFLOP/s", frac=round(achieved / peak, 4),
                frac_of={k: round(achieved / v, 4) for k, v in others.items()},
                peaks_of={k: v for k, v in others.items()})


def traffic_from_profiles(name):
    """HBM bytes per launch of the config's dominant kernel, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary tagged `bench_config: <name>`, if one exists."""
    for p in sorted((ROOT / "profiles").glob("*_pmc.md")):
        text = p.read_text()
        if not re.search(rf"^bench_config:\s*{re.escape(name)}\s*$", text, re.M):
            continue
        m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", text)
        if m:
            return float(m.group(1))
    return None


def host_threads():
    """Host threads the CPU baseline may use, and how that number was found.

    The job's CPU share is the smallest of the affinity mask, the cgroup CPU
    quota and OMP_NUM_THREADS (a host that shares its CPUs among one-GPU jobs
    grants each a fixed share and sets OMP_NUM_THREADS to it); os.cpu_count()
    is reported beside it."""
    n_aff = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    limits = {"affinity": n_aff}
    try:
        q, p = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if q != "max":
            limits["cgroup_quota"] = max(1, int(int(q) // int(p)))
    except (OSError, ValueError):
        pass
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        limits["OMP_NUM_THREADS"] = max(1, int(os.environ["OMP_NUM_THREADS"]))
    used = min(limits.values())
    return used, dict(limits, os_cpu_count=os.cpu_count())


def cpu_baseline(cfg, xb, wq, s, budget_s=4.0):
    """Oracle's fp32-accumulating qmm on every host thread of the job's CPU share,
    over a bounded sample of the workload."""
    import oracle as O

    threads, limits = host_threads()
    M, N, K = cfg["M"], cfg["N"], cfg["K"]
    rows = N
    # for the compute-bound configs take a slice of output columns (full K, all M rows)
    if M > 8:
        rows = max(64, min(N, int(N * 0.004)))
    w_s, s_s = wq[:rows], s[:rows]
    t0 = time.perf_counter()
    O.qmm(cfg["mode"], xb, w_s, s_s, f32acc=True, threads=threads)
    one = time.perf_counter() - t0
    reps = max(1, min(1000, int(budget_s / max(one, 1e-6))))
    t0 = time.perf_counter()
    for _ in range(reps):
        O.qmm(cfg["mode"], xb, w_s, s_s, f32acc=True, threads=threads)
    dt = (time.perf_counter() - t0) / reps
    sample_cfg = dict(cfg, N=rows)
    alg = algorithmic(sample_cfg)
    if M <= 8:
        value, unit = alg["bytes"] / dt / 1e9, "GB/s"
    else:
        value, unit = alg["flops"] / dt / 1e12, "TFLOP/s"
    share = ", ".join(f"{k}={v}" for k, v in limits.items())
    sample = (f"{reps} calls of M={M} x {rows} of {N} output rows, K={K} ({cfg['mode']}), "
              f"{dt * 1e3:.2f} ms/call, {reps * dt:.1f} s total; CPU restatement (not MLX) on {threads} threads "
              f"= the job's CPU share ({share})")
    return dict(value=round(value, 4), unit=unit, cores=threads, kind="port", sample=sample,
                us_per_call=round(dt * 1e6, 1))


def gdn_bytes(cfg):
    """Algorithmic bytes of one GDN call: state in and out (f32), q, k, v, y (bf16), g (f32), beta (bf16)."""
    B, T, Hk, Hv, Dk, Dv = (cfg[k] for k in ("B", "T", "Hk", "Hv", "Dk", "Dv"))
    return 2 * 4 * B * Hv * Dv * Dk + 2 * 2 * B * T * Hk * Dk + 2 * 2 * B * T * Hv * Dv + (4 + 2) * B * T * Hv


def gdn_flops(cfg):
    """Per step and state row: decay (Dk mul), two dot products and the update (3 Dk FMA)."""
    B, T, Hv, Dk, Dv = (cfg[k] for k in ("B", "T", "Hv", "Dk", "Dv"))
    return B * T * Hv * Dv * 7 * Dk


def queued_timed(step, steps, reps=5):
    """K eager launches queued behind a GPU sleep (ms per call, the median of `reps`), or
    None when the host's enqueueing of the K launches outlasted the sleep once."""
    import statistics

    import torch

    import qmm as Q

    if not hasattr(torch.cuda, "_sleep"):  # (torch's spin kernel; absent: time a graph replay)
        return None
    st = Q.Stream.torch_current()
    t0, launches, host = time.perf_counter(), 0, []
    while True:  # untimed batches until the clocks hold: at least 1 s and 2000 launches (at most 3 s)
        h0 = time.perf_counter()
        for i in range(steps):
            step(i, st)
        host.append((time.perf_counter() - h0) / steps)
        torch.cuda.synchronize()
        launches += steps
        spent = time.perf_counter() - t0
        if (spent >= 1.0 and launches >= 2000) or spent > 3.0:
            break
    # a sleep of at least twice the host's median enqueueing time for K launches (the spin
    # kernel counts shader clocks, at most 2.5 GHz here, so this many cycles last at least that)
    cycles = int((2.0 * statistics.median(host) * steps + 2e-4) * 2.5e9)
    res = []
    for _ in range(reps):
        a, s, e = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        a.record()
        torch.cuda._sleep(cycles)
        s.record()
        h0 = time.perf_counter()
        for i in range(steps):
            step(i, st)
        host_ms = (time.perf_counter() - h0) * 1e3
        e.record()
        e.synchronize()
        if host_ms >= a.elapsed_time(s):
            return None  # the first kernels may have waited for the host
        res.append(s.elapsed_time(e) / steps)
    return statistics.median(res)


def timed(step, steps, args):
    """ms per call and how it was timed (args.graph / args.no_graph pick a method)."""
    import torch

    import qmm as Q

    if getattr(args, "no_graph", False):
        st = Q.Stream.torch_current()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for i in range(steps):
            step(i, st)
        end.record()
        end.synchronize()
        return start.elapsed_time(end) / steps, "eager"
    if not getattr(args, "graph", False):
        ms = queued_timed(step, steps)
        if ms is not None:
            return ms, "eager launches queued behind a GPU sleep (median of 5)"
    return replay_timed(step, steps), "hip graph replay"


def replay_timed(step, steps):
    """Capture `steps` calls in a HIP graph, settle the clocks, time one replay (ms per call)."""
    import torch

    import qmm as Q

    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        step(0, Q.Stream.torch_current())
        torch.cuda.current_stream().synchronize()
        with torch.cuda.graph(g, stream=cap):
            for i in range(steps):
                step(i, Q.Stream.torch_current())
    torch.cuda.synchronize()
    # Untimed replays bring the clocks to their steady state under this load: at least
    # 1 s and 2000 launches (measured: a 20-launch graph timed right after capture reads
    # ~4% slow), then until two consecutive replays agree within 2% (at most 3 s).
    t0 = time.perf_counter()
    launches, prev = 0, None
    while True:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        e1.synchronize()
        launches += steps
        cur = e0.elapsed_time(e1)
        spent = time.perf_counter() - t0
        settled = prev is not None and abs(cur - prev) <= 0.02 * prev
        if (spent >= 1.0 and launches >= 2000 and settled) or spent > 3.0:
            break
        prev = cur
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    # The timed replay is queued behind an untimed one: the host submits it while the
    # GPU runs the first, so the start event fires when the first replay's last kernel
    # ends and the K timed launches follow it back to back.  Recorded on an idle stream
    # instead, the start event would also time the host's graph submission, which at
    # K = 20 adds ~0.5 us per call.
    g.replay()
    start.record()
    g.replay()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / steps


def bench_gdn(args, cfg):
    """The GDN recurrence (qmm_gdn_recurrence): states rotate over >= 512 MiB of copies so each
    call reads its state from HBM; each call updates its state in place."""
    import numpy as np
    import torch

    import qmm as Q

    B, T, Hk, Hv, Dk, Dv = (cfg[k] for k in ("B", "T", "Hk", "Hv", "Dk", "Dv"))
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    rn = lambda *s: torch.randn(s, generator=gen, device=dev, dtype=torch.float32)
    q = rn(B, T, Hk, Dk)
    k = rn(B, T, Hk, Dk)
    q = (q / q.pow(2).mean(-1, keepdim=True).sqrt() / Dk).to(torch.bfloat16)
    k = (k / k.pow(2).mean(-1, keepdim=True).sqrt() / math.sqrt(Dk)).to(torch.bfloat16)
    v = rn(B, T, Hv, Dv).to(torch.bfloat16)
    g = torch.exp(-0.35 * torch.rand((B, T, Hv), generator=gen, device=dev))
    beta = torch.sigmoid(rn(B, T, Hv)).to(torch.bfloat16)
    sbytes = 4 * B * Hv * Dv * Dk
    copies = max(1, math.ceil(ROTATE_BYTES / sbytes))
    states = [Q.Array.from_torch(rn(B, Hv, Dv, Dk) * 0.1) for _ in range(copies)]
    yt = torch.empty((B, T, Hv, Dv), dtype=torch.bfloat16, device=dev)
    A = Q.Array.from_torch
    qa, ka, va, ga, ba, ya = A(q), A(k), A(v), A(g), A(beta), A(yt)
    torch.cuda.synchronize()
    print(f"[bench] {args.config}: {cfg['workload']}; {copies} state copies, steps={args.steps} "
          f"warmup={args.warmup}", file=sys.stderr, flush=True)

    def step(i, st):
        s_i = states[i % copies]
        Q.gdn_recurrence(qa, ka, va, ga, ba, s_i, y=ya, state_out=s_i, stream=st)

    for i in range(args.warmup):
        step(i, Q.Stream.torch_current())
    torch.cuda.synchronize()
    ms, how = timed(step, args.steps, args)
    nbytes, flops = gdn_bytes(cfg), gdn_flops(cfg)
    achieved = nbytes / (ms / 1e3) / 1e9
    roof = dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                frac=round(achieved / HBM_PEAK_GBS, 4), traffic=traffic_from_profiles(args.config))
    cpu = None
    if not args.no_cpu:
        from gdn import gdn_recurrence  # the oracle, timed on the host as the CPU baseline

        f = lambda t_: t_.float().cpu().numpy()
        Ts = min(T, 8)
        s0 = states[0].numpy()
        t0 = time.perf_counter()
        reps = 0
        while True:
            gdn_recurrence(f(q[:, :Ts]), f(k[:, :Ts]), f(v[:, :Ts]), f(g[:, :Ts]), f(beta[:, :Ts]), s0, acc="f32")
            reps += 1
            if time.perf_counter() - t0 > 3.0:
                break
        sec_step = (time.perf_counter() - t0) / (reps * Ts)
        cpu_sec = sec_step * T
        cpu = {"value": round(nbytes / cpu_sec / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"{reps} runs of {Ts} of the {T} steps (numpy float32, one thread of vector ops), "
                         f"scaled to {T} steps: {cpu_sec * 1e3:.2f} ms/call"}
    line = {
        "metric": "GDN recurrence GB/s & % HBM peak (state + inputs + y per call)", "value": roof["achieved"],
        "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "us_per_call": round(ms * 1e3, 2), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 state, bf16 q/k/v/beta/y", "data": "synthetic (seeded; RMS-normalised q, k as the model feeds)",
        "config": {"workload": cfg["workload"], "B": B, "T": T, "Hk": Hk, "Hv": Hv, "Dk": Dk, "Dv": Dv,
                   "state_copies": copies, "algorithmic_bytes": nbytes, "algorithmic_flops": flops,
                   "gflops": round(flops / (ms / 1e3) / 1e9, 1), "timing": how},
        "roofline": roof, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def bench_census(args):
    """Time every call-site shape of one decoded token (CENSUS) in one mode at M rows.

    Each shape's quantized weights are replicated at 256-byte aligned offsets of one
    buffer of >= 512 MiB (one copy if larger), so every timed call reads cold weights
    even for the 48-row projections.  mxfp8 checkpoints keep lm_head dense bf16
    (src/model.zig:215-216), so in mxfp8 mode lm_head runs the dense GEMV.  Prints one
    JSON line: per-shape us, GB/s and fraction of HBM peak, and the per-token sums with
    gate and up as two calls or as the fused gate+up+SiLU*mul call."""
    import numpy as np
    import torch

    import qmm as Q

    mode, M = args.census, args.census_m
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    stream = Q.Stream.torch_current()
    al = lambda n: (n + 255) // 256 * 256
    gen.manual_seed(7)
    x_full = (torch.randn((M, 17408), generator=gen, device=dev, dtype=torch.float32)).to(torch.bfloat16)
    rows = [(name, N, K, calls, site, False, None) for name, N, K, calls, site in CENSUS]
    rows.append(("mlp.gate_up_silu (fused gate+up)", 17408, 5120, 64, "src/model.zig:905-915", True, None))
    # grouped projections of one x (qmm_quantized_matmul_group), members back to back
    for gname, members in CENSUS_GROUPS.items():
        parts = [r for r in CENSUS if r[0] in members]
        rows.append((gname, sum(r[1] for r in parts), parts[0][2], parts[0][3],
                     ", ".join(r[4] for r in parts), False, [r[1] for r in parts]))
    results = []
    for name, N, K, calls, site, fused, group in rows:
        m = "bf16" if (mode == "mxfp8" and name == "lm_head") else mode
        gen.manual_seed(1000 + N + K)
        W = (torch.randn((N, K), generator=gen, device=dev, dtype=torch.float32) * 0.02).to(torch.bfloat16)
        if m == "bf16":
            parts = [W.contiguous().view(torch.uint8).view(-1)]
        else:
            wq, sc = Q.quantize(Q.Array.from_torch(W), m, stream=stream)
            torch.cuda.synchronize()
            parts = [torch.from_numpy(a.numpy().view(np.uint8).reshape(-1)).to(dev) for a in (wq, sc)]
            del wq, sc
        del W
        sizes = [p.numel() for p in parts]
        per = sum(al(s) for s in sizes)
        copies = max(2 if fused else 1, math.ceil(ROTATE_BYTES / per))
        buf = torch.empty(copies * per, dtype=torch.uint8, device=dev)
        mats, tmats = [], []
        for c in range(copies):
            off, views = c * per, []
            for p, s in zip(parts, sizes):
                buf[off:off + s].copy_(p)
                views.append(buf[off:off + s])
                off += al(s)
            if m == "bf16":
                mats.append((Q.Array.from_torch(views[0].view(torch.bfloat16).view(N, K)),))
            else:
                wcols = K * BITS[m] // 32
                tmats.append((views[0].view(torch.int32).view(N, wcols), views[1].view(N, K // GROUP[m])))
                mats.append((Q.Array.from_torch(tmats[-1][0], dtype=Q.UINT32), Q.Array.from_torch(tmats[-1][1])))
        del parts
        x = Q.Array.from_torch(x_full[:, :K].contiguous())
        yt = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        y = Q.Array.from_torch(yt)
        torch.cuda.synchronize()

        if group:
            # each copy's members: row slices of the copy (back to back, as the loader places them)
            gmats, outs = [], [Q.Array.from_torch(torch.empty((M, n), dtype=torch.bfloat16, device=dev))
                               for n in group]
            for wt_, st_ in tmats:
                ws_, ss_, r0 = [], [], 0
                for n in group:
                    ws_.append(Q.Array.from_torch(wt_[r0:r0 + n], dtype=Q.UINT32))
                    ss_.append(Q.Array.from_torch(st_[r0:r0 + n]))
                    r0 += n
                gmats.append((ws_, ss_))

        def step(i, st):
            if group:
                ws_, ss_ = gmats[i % copies]
                Q.quantized_matmul_group(x, ws_, ss_, m, outs=outs, stream=st)
            elif fused:
                (wg, sg), (wu, su) = mats[i % copies], mats[(i + 1) % copies]
                Q.mlp_gate_up_silu(x, wg, sg, wu, su, m, out=y, stream=st)
            elif m == "bf16":
                Q.linear(x, mats[i % copies][0], out=y, stream=st)
            else:
                wq_, sc_ = mats[i % copies]
                Q.quantized_matmul(x, wq_, sc_, m, out=y, stream=st)

        for i in range(max(args.warmup, copies)):  # every weight copy once (its prefill scale copy)
            step(i, stream)
        torch.cuda.synchronize()
        ms, how = timed(step, args.steps, args)
        cfg = dict(mode=m, M=M, N=N, K=K, mlp=fused)
        alg = algorithmic(cfg)
        gbs = alg["bytes"] / (ms / 1e3) / 1e9
        results.append(dict(weight=name, site=site, mode=m, N=N, K=K, calls_per_token=calls,
                            us=round(ms * 1e3, 2), gbs=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4),
                            bytes=alg["bytes"], copies=copies))
        print(f"[census] {name:34s} {m:5s} N={N:6d} K={K:5d} M={M}: {ms * 1e3:8.2f} us {gbs:7.1f} GB/s "
              f"({gbs / HBM_PEAK_GBS:.3f})", file=sys.stderr, flush=True)
        del mats, tmats, buf, x, y, yt
        if group:
            del gmats, outs
        torch.cuda.empty_cache()
    extra = ("mlp.gate_up_silu",) + tuple(CENSUS_GROUPS)
    base = [r for r in results if not r["weight"].startswith(extra)]
    by = {r["weight"]: r for r in results}
    us_sep = sum(r["us"] * r["calls_per_token"] for r in base)
    bytes_sep = sum(r["bytes"] * r["calls_per_token"] for r in base)
    cost = lambda names: sum(by[n]["us"] * by[n]["calls_per_token"] for n in names)
    us_fused = us_sep - cost(("mlp.gate_proj", "mlp.up_proj")) + cost(("mlp.gate_up_silu (fused gate+up)",))
    us_grouped = us_fused
    for gname, members in CENSUS_GROUPS.items():
        us_grouped += cost((gname,)) - cost(members)
    line = {
        "census": mode, "M": M, "steps": args.steps, "timing": f"per shape: {how}",
        "data": "synthetic (seeded N(0,1) x, N(0,0.02) W quantized on device)",
        "shapes": results,
        "per_token": {"calls": sum(r["calls_per_token"] for r in base), "weight_bytes": bytes_sep,
                      "us_separate": round(us_sep, 1), "us_mlp_fused": round(us_fused, 1),
                      "us_mlp_fused_and_grouped": round(us_grouped, 1),
                      "gbs_separate": round(bytes_sep / us_sep / 1e3, 1),
                      "gbs_mlp_fused_and_grouped": round(bytes_sep / us_grouped / 1e3, 1)},
    }
    print(json.dumps(line), flush=True)


# The workloads the headline metric is quoted on, in the order the default run
# times them; the first is the headline `value`.
HEADLINE_SET = ["gateup", "mxfp8_gemv", "down_m1", "down_m2", "down_m3", "prefill", "lmhead", "lmhead_prefill"]
METRIC = "qmatmul GB/s & % HBM peak at M=1 (nvfp4/mxfp8); TFLOPS & % MFMA at M=4096"


def make_weights(cfg, copies, Q, torch, stream, dev):
    """`copies` distinct seeded weight matrices of the config, quantized on the device."""
    mode, N, K = cfg["mode"], cfg["N"], cfg["K"]
    gen = torch.Generator(device=dev)
    weights = []
    for r in range(copies):
        gen.manual_seed(1000 + r)
        W = (torch.randn((N, K), generator=gen, device=dev, dtype=torch.float32) * 0.02).to(torch.bfloat16)
        if mode == "bf16":
            weights.append((Q.Array.from_torch(W), None))
            continue
        wq, sc = Q.quantize(Q.Array.from_torch(W), mode, stream=stream)
        del W
        if cfg.get("mlp"):
            gen.manual_seed(2000 + r)
            W2 = (torch.randn((N, K), generator=gen, device=dev, dtype=torch.float32) * 0.02).to(torch.bfloat16)
            wq2, sc2 = Q.quantize(Q.Array.from_torch(W2), mode, stream=stream)
            weights.append((wq, sc, wq2, sc2))
            del W2
            continue
        weights.append((wq, sc))
    return weights


def measure_qmm(name, args, cache):
    """Time one quantized-linear config; returns its result dict (the JSON line's fields)."""
    import numpy as np
    import torch

    import qmm as Q

    cfg = CONFIGS[name]
    mode, M, N, K = cfg["mode"], cfg["M"], cfg["N"], cfg["K"]
    alg = algorithmic(cfg)
    torch.cuda.set_device(0)
    dev = torch.device("cuda", 0)
    copies = max(1, math.ceil(ROTATE_BYTES / (alg["w"] + alg["s"])))
    stream = Q.Stream.torch_current()
    key = (mode, N, K, bool(cfg.get("mlp")), copies)
    if cache.get("key") != key:  # configs on the same weights (lm_head decode and prefill) share them
        cache.clear()
        torch.cuda.empty_cache()
        cache["key"], cache["weights"] = key, make_weights(cfg, copies, Q, torch, stream, dev)
    weights = cache["weights"]
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    xt = (torch.randn((M, K), generator=gen, device=dev, dtype=torch.float32) * cfg["xscale"]).to(torch.bfloat16)
    x = Q.Array.from_torch(xt)
    yt = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    y = Q.Array.from_torch(yt)
    torch.cuda.synchronize()
    print(f"[bench] {name}: {cfg['workload']}; {copies} weight copies, steps={args.steps} "
          f"warmup={args.warmup}", file=sys.stderr, flush=True)

    def step(i, st):
        if cfg.get("mlp"):
            wg, sg, wu, su = weights[i % copies]
            Q.mlp_gate_up_silu(x, wg, sg, wu, su, mode, out=y, stream=st)
            return
        wq, sc = weights[i % copies]
        if mode == "bf16":
            Q.linear(x, wq, out=y, stream=st)
        else:
            Q.quantized_matmul(x, wq, sc, mode, out=y, stream=st)

    # untimed: at least W steps, and one call on every weight copy (a prefill call's first use
    # of a scales handle makes its tile-major copy; a graph captured before that would
    # repack those scales on every replay)
    for i in range(max(args.warmup, copies)):
        step(i, stream)
    torch.cuda.synchronize()

    ms, how = timed(step, args.steps, args)
    roof = roofline_of(cfg, alg, ms / 1e3)
    roof["traffic"] = traffic_from_profiles(name)

    cpu = None
    if not args.no_cpu and mode != "bf16" and not cfg.get("mlp"):
        wq0, sc0 = weights[0]
        cpu = cpu_baseline(cfg, xt.view(torch.int16).cpu().numpy().view(np.uint16), wq0.numpy(), sc0.numpy(),
                           budget_s=args.cpu_budget)
    print(f"[bench] {name}: {ms * 1e3:.2f} us/call, {roof['achieved']} {roof['unit']} ({roof['frac']:.3f} of "
          f"{roof['peak']:.0f})" + (f"; CPU {cpu['value']} {cpu['unit']} on {cpu['cores']} threads" if cpu else ""),
          file=sys.stderr, flush=True)
    return {
        "name": name, "ms_per_step": round(ms, 5), "us_per_call": round(ms * 1e3, 2),
        "dtype": "bf16 (fp32 accumulate)" if mode == "bf16" else f"{mode} weights x bf16 (fp32 accumulate)",
        "config": {"workload": cfg["workload"], "mode": mode, "M": M, "N": N, "K": K, "weight_copies": copies,
                   "algorithmic_bytes": alg["bytes"], "algorithmic_flops": alg["flops"],
                   "timing": how},
        "roofline": roof, "cpu_baseline": cpu,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default=None, choices=sorted(CONFIGS),
                    help="time one workload (default: every headline workload, the gate+up GEMV first)")
    ap.add_argument("--no-graph", action="store_true", help="time unqueued eager launches")
    ap.add_argument("--graph", action="store_true", help="time one HIP graph replay of the K calls")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-budget", type=float, default=4.0, help="seconds of CPU baseline per workload")
    ap.add_argument("--census", choices=("nvfp4", "mxfp8"),
                    help="instead of one config, time every quantized linear of a decoded token in this mode")
    ap.add_argument("--census-m", type=int, default=1, help="x rows for --census (1 decode, 2-3 MTP verify)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="instead of the workload, run K plain 512 MiB -> 512 MiB copy kernels (torch.neg on "
                         "float32) so HBM counters (FETCH_SIZE / WRITE_SIZE) can be scaled to known bytes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this path runs on a single MI355X); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import qmm as Q  # noqa: F401  (loads libqmm.so; fails loudly if it is not built)

    if args.copy_calibration:
        n = 128 << 20  # float32 elements: 512 MiB read + 512 MiB written per launch
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(args.steps):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        print(json.dumps({"copy_kernel": "torch.neg float32", "bytes_read_per_launch": n * 4,
                          "bytes_written_per_launch": n * 4, "launches": args.steps}), flush=True)
        return

    if args.census:
        return bench_census(args)
    if args.config and CONFIGS[args.config].get("gdn"):
        return bench_gdn(args, CONFIGS[args.config])
    names = [args.config] if args.config else HEADLINE_SET
    cache = {}
    results = [measure_qmm(n, args, cache) for n in names]
    cache.clear()
    head = results[0]
    line = {
        "metric": METRIC, "value": head["roofline"]["achieved"], "unit": head["roofline"]["unit"], "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": head["ms_per_step"],
        "us_per_call": head["us_per_call"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": head["dtype"], "data": "synthetic (seeded N(0,1) x, N(0,0.02) W quantized on device)",
        "config": head["config"], "roofline": head["roofline"], "cpu_baseline": head["cpu_baseline"],
    }
    if len(results) > 1:
        line["configs"] = [{k: r[k] for k in ("name", "us_per_call", "dtype", "config", "roofline", "cpu_baseline")}
                           for r in results]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
