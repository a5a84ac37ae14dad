#!/usr/bin/env python3
"""Benchmark of the SimSD matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2]

Workloads (synthetic data, bf16, random-init weights of the named shapes):
  c2      default: the SDAR-1.7B-shape draft linear set at M=4 -- 28 layers x
          {qkv 2048->4096, o 2048->2048, gate_up 2048->12288, down 6144->2048},
          weights ~N(0, 0.02) with a fresh seed per layer, activations ~N(0, 1).
          One step = the 112 linears once (2.83 GB of weights, > the 256 MB MALL).
  c1      the merged gate_up 2048->12288 at M=4 alone, cycled over 24 distinct
          weights (1.2 GB) so the MALL cannot serve repeats.
  c3m16 / c3m32
          8B-shape target verify set, 36 layers x {qkv 4096->6144, o 4096->4096,
          gate_up 4096->24576, down 12288->4096} + lm_head 4096->151936, M=16/32.
  mlp4 / mlp16 / mlp32
          the gated MLP block per layer (28 draft layers at M=4, 36 target
          layers at M=16/32): gate and up projections with SiLU-mul fused
          (thin_linear_silu_mul), then down; also times the unfused sequence.
  layer4 / layer16 / layer32 / layer36 / layer48
          the linear path of each decoder layer with the fused epilogues
          (36 and 48 rows: the verify with one or four committed blocks
          folded in):
          RMSNorm + qkv, o, RMSNorm + gate/up + SiLU-mul, down (four launches;
          six above 8 tokens, where each norm is a launch of its own),
          against the unfused sequence with the stock PyTorch RMSNorm.
  head4 / head32
          the lm_head with its epilogue: the draft's denoise step on a 4-token
          block (lm_head 2048->151936, softmax/argmax/confidence, masked
          unmasking) and the target's verify pass over 32 rows (lm_head
          4096->151936, softmax probabilities of the 16 mask rows), fused
          against the reference's torch sequence.
  attn4 / attn32
          attention of the block over the static KV cache per layer: q/k norm +
          RoPE + cache write, then attention over 1024 slots (28 draft layers,
          4 rows, 16/8 heads; 36 target layers, 32 rows, 32/8 heads), against
          the reference's sequence on its GQA-expanded cache.  --context sets
          the valid slots (up to 4096) for a sweep over lengths.
  verify36
          the target's verify forward as the runner issues it: random-init
          SDAR-8B shape, 36 rows (one committed block folded in + 4 blocks of
          4 data and 4 mask rows) over a 1024-slot context, lm_head on the 16
          mask rows; the projections' split-K partials summed by the launches
          consuming them, against the reduce-first form.
  c5      the end-to-end speculative step: random-init SDAR-1.7B draft and
          SDAR-8B target on one GPU, 512-token prompt, 4-token blocks, 4
          denoise steps, 4 blocks verified per target forward, greedy
          acceptance; value in generated tokens / s.
  copy    a plain 1 GiB device copy: calibrates the PMC byte counters.
  c4t4 / c4t16 / c4t64
          MoE step (route top-8 softmax over 256 experts -> align -> grouped
          gate_up + SiLU.mul -> down -> combine, + one shared expert),
          H=2048, I=512, T tokens; cycled over 8 distinct layers.
Each step is captured once in a HIP graph and replayed; the timed region is
K replays bracketed by synchronisations and HIP events on the replay stream.
The default run (c2) also times c1, c3m16, c3m32, c4t4, c4t16, c4t64 and c5,
each in a child process of its own, and adds them under "extras" in the same
JSON line (--no-extras skips them); progress goes to stderr.

value = algorithmic bytes per step / time per step (weights read once +
activations in + outputs out).  The roofline object is for the dominant
kernel; every launch in the c1/c2/c3 timed region is that kernel, so its
average launch duration is the region time / launches.  "traffic" is the
HBM bytes per launch from the committed rocprofv3 PMC summary under
profiles/ for the workload (null if none).  "breakdown" times each op's
calls alone in a graph of their own.  The CPU baseline is the reference's CPU path -- torch
F.linear in bf16 (its oracle ref_thin_linear), the stock MoE loop, or (c5)
the reference's decoder layer forward -- timed on a bounded sample of the
same workload; every extra of the default run carries its own.
"""
from __future__ import annotations

import argparse
import glob
import json
import os
import re
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.join(REPO, "simsd-release_amd"))

METRIC = "skinny-GEMM HBM GB/s (% of peak) at M=4/16/32; spec-decode tok/s on 1 GPU"
HBM_PEAK_GBS = 8000.0
BF16 = 2

DRAFT = [("qkv", 2048, 4096), ("o", 2048, 2048), ("gate_up", 2048, 12288), ("down", 6144, 2048)]
TARGET = [("qkv", 4096, 6144), ("o", 4096, 4096), ("gate_up", 4096, 24576), ("down", 12288, 4096)]
LM_HEAD_TARGET = ("lm_head", 4096, 151936)


def linear_bytes(M, K, N):
    return N * K * BF16 + M * K * BF16 + M * N * BF16


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def measured_traffic(workload: str):
    """HBM bytes per launch of the dominant kernel for this workload (per
    step for the MoE step, whose roofline is per step), as recorded in a
    committed rocprofv3 PMC summary under profiles/ (FETCH_SIZE + WRITE_SIZE
    per dispatch, scaled by a plain copy kernel's reading); None when no
    summary covers the workload."""
    pat = re.compile(r"^traffic_bytes_per_(?:launch|step):\s*(\w+)\s*=\s*(\d+)")
    for path in sorted(glob.glob(os.path.join(REPO, "profiles", "*.md"))):
        for line in open(path):
            m = pat.match(line.strip())
            if m and m.group(1) == workload:
                return int(m.group(2))
    return None


# ───────────────────────────────────────────────────────────── workloads ───
def make_linear_calls(torch, dev, workload):
    """[(op name, x, w)] for one step."""
    calls = []

    def rand(shape, scale, seed):
        g = torch.Generator(device=dev).manual_seed(seed)
        return (torch.randn(*shape, generator=g, device=dev, dtype=torch.float32) * scale).to(torch.bfloat16)

    if workload == "c2":
        M = 4
        for layer in range(28):
            for j, (name, K, N) in enumerate(DRAFT):
                seed = 1000 + layer * 16 + j
                calls.append((name, rand((M, K), 1.0, seed), rand((N, K), 0.02, seed + 100000)))
        return M, calls
    if workload == "c1":
        M, K, N = 4, 2048, 12288
        for i in range(24):
            calls.append(("gate_up", rand((M, K), 1.0, 50 + i), rand((N, K), 0.02, 5000 + i)))
        return M, calls
    if workload in ("c3m16", "c3m32"):
        M = 16 if workload == "c3m16" else 32
        for layer in range(36):
            for j, (name, K, N) in enumerate(TARGET):
                seed = 2000 + layer * 16 + j
                calls.append((name, rand((M, K), 1.0, seed), rand((N, K), 0.02, seed + 100000)))
        name, K, N = LM_HEAD_TARGET
        calls.append((name, rand((M, K), 1.0, 7), rand((N, K), 0.02, 8)))
        return M, calls
    raise ValueError(workload)


def graph_us_per_call(torch, fns, reps=20):
    """Capture fns (no-arg launches) in one graph; replay; us per launch."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for f in fns:
            f()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fns:
            f()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps / len(fns)


def cpu_baseline_linear(torch, workload, M):
    """torch CPU F.linear (bf16) on a bounded sample: 4 distinct layers of the
    workload's shapes, cycled to one full step."""
    from oracle.thin_linear import linear_cpu_torch

    shapes = DRAFT if workload in ("c2", "c1") else TARGET
    n_layers = {"c2": 28, "c1": 0}.get(workload, 36)
    if workload == "c1":
        shapes = [("gate_up", 2048, 12288)]
    g = torch.Generator().manual_seed(0)
    sample_layers = 4 if workload != "c1" else 8

    def pair(K, N):
        # uniform weights of the same spread as N(0, 0.02): a CPU GEMM's time
        # does not depend on the values, and filling gigabytes is faster
        return (torch.randn(M, K, generator=g).to(torch.bfloat16),
                torch.empty(N, K, dtype=torch.bfloat16).uniform_(-0.0346, 0.0346, generator=g))

    layers = [[pair(K, N) for _, K, N in shapes] for _ in range(sample_layers)]
    per_layer_bytes = sum(linear_bytes(M, K, N) for _, K, N in shapes)
    step_layers = n_layers if n_layers else 24
    # the target verify set ends with its lm_head, once per step
    head = pair(*LM_HEAD_TARGET[1:]) if workload in ("c3m16", "c3m32") else None

    def step():
        for i in range(step_layers):
            for x, w in layers[i % sample_layers]:
                linear_cpu_torch(x, w)
        if head is not None:
            linear_cpu_torch(*head)

    step()                                  # warmup
    times = []
    t_end = time.perf_counter() + 12.0
    while len(times) < 20 and (time.perf_counter() < t_end or len(times) < 3):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    byts = per_layer_bytes * step_layers + (linear_bytes(M, *LM_HEAD_TARGET[1:]) if head is not None else 0)
    return {
        "value": round(byts / med / 1e9, 3),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"torch CPU F.linear bf16 (the reference oracle ref_thin_linear), M={M}, "
                   f"{sample_layers} distinct layers of {[s[0] for s in shapes]} "
                   f"({sample_layers * per_layer_bytes / 1e6:.0f} MB of weights) cycled to one "
                   f"{step_layers}-layer step{' + the lm_head' if head is not None else ''}; median of "
                   f"{len(times)} steps ({med * 1e3:.1f} ms/step); cpu={cpu_model()}; "
                   f"os.cpu_count={os.cpu_count()}"),
    }


def run_linear(args, torch, dev):
    from kernels.thin_linear_fused import thin_linear

    M, calls = make_linear_calls(torch, dev, args.workload)
    step_bytes = sum(linear_bytes(M, x.shape[1], w.shape[0]) for _, x, w in calls)
    launches = len(calls)

    def step():
        return [thin_linear(x, w) for _, x, w in calls]

    with torch.inference_mode():
        # eager warmup: allocates the split-K workspace before capture
        for _ in range(2):
            step()
        torch.cuda.synchronize()
        # per-op time: each op's calls alone in a graph of their own
        per_op = {}
        for name in dict.fromkeys(n for n, _, _ in calls):
            mine = [(x, w) for n, x, w in calls if n == name]
            us = graph_us_per_call(torch, [lambda x=x, w=w: thin_linear(x, w) for x, w in mine])
            K, N = mine[0][0].shape[1], mine[0][1].shape[0]
            per_op[name] = {"K": K, "N": N, "calls": len(mine), "us": us,
                            "bytes": linear_bytes(M, K, N)}

        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(args.steps):
            graph.replay()
        t1.record(stream)
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / args.steps
        floor = None
        if args.workload == "c1":
            # the same 24 weights read by library kernels, for the floor of
            # one launch streaming 48 MiB: torch's sum (reads the weight,
            # writes one value) and a device copy (reads and writes it)
            sink = torch.empty(len(calls), dtype=torch.float32, device=dev)
            dst = torch.empty_like(calls[0][2])
            sum_us = graph_us_per_call(torch, [lambda i=i, w=w: torch.sum(w, dim=(0, 1), dtype=torch.float32, out=sink[i])
                                               for i, (_, _, w) in enumerate(calls)])
            copy_us = graph_us_per_call(torch, [lambda w=w: dst.copy_(w) for _, _, w in calls])
            floor = {"sum_us_per_weight": round(sum_us, 3), "copy_us_per_weight": round(copy_us, 3),
                     "weight_bytes": calls[0][2].numel() * BF16,
                     "note": "library kernels over the same 24 weights in a graph: torch.sum reads 48 MiB, "
                             "a device copy reads and writes it"}

    gbs = step_bytes / (ms * 1e-3) / 1e9
    avg_launch_us = ms * 1e3 / launches
    kernel = ("thin_gemv4_kernel (4x4x4 MFMA GEMV, M <= 8)" if M <= 8 else
              "thin_gemm_lds_kernel (16x16x32 MFMA via LDS; per call, the split-K reduce "
              "launch of down_proj included)")
    breakdown = {
        n: {"K": d["K"], "N": d["N"], "calls": d["calls"], "us_per_call": round(d["us"], 3),
            "GB/s": round(d["bytes"] / (d["us"] * 1e-6) / 1e9, 1),
            "frac": round(d["bytes"] / (d["us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        for n, d in per_op.items()}
    result = {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": {"c2": "draft-linear-set-M4-28L", "c1": "gate_up-2048x12288-M4",
                                "c3m16": "target-verify-set-M16-36L+lm_head",
                                "c3m32": "target-verify-set-M32-36L+lm_head"}[args.workload],
                   "M": M, "launches_per_step": launches, "algorithmic_bytes_per_step": step_bytes,
                   "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": round(step_bytes / launches / (avg_launch_us * 1e-6) / 1e9, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(step_bytes / launches / (avg_launch_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(args.workload),
                     "kernel": kernel,
                     "bytes_per_launch": round(step_bytes / launches),
                     "avg_launch_us": round(avg_launch_us, 3)},
        "breakdown": breakdown,
        "tflops": round(sum(2 * M * x.shape[1] * w.shape[0] for _, x, w in calls) / (ms * 1e-3) / 1e12, 2),
    }
    if floor is not None:
        result["library_read_floor"] = floor
    return result, M


# ─────────────────────────────────────────────────────── gated MLP block ───
def run_mlp(args, torch, dev):
    """The MLP half of each layer: h = silu(x Wg^T) * (x Wu^T) in one kernel,
    then down.  Also times the unfused sequence (merged gate_up linear,
    PyTorch SiLU and product, down) on the same weights."""
    from kernels.thin_linear_fused import thin_linear, thin_linear_silu_mul

    M = {"mlp4": 4, "mlp16": 16, "mlp32": 32}[args.workload]
    H, I, L = (2048, 6144, 28) if M == 4 else (4096, 12288, 36)
    layers = []
    for layer in range(L):
        g = torch.Generator(device=dev).manual_seed(4000 + layer)
        mk = lambda *sh, s=1.0: (torch.randn(*sh, device=dev, generator=g) * s).to(torch.bfloat16)
        layers.append((mk(M, H), mk(2 * I, H, s=0.02), mk(H, I, s=0.02)))
    step_bytes = L * (2 * I * H * 2 + H * I * 2 + M * H * 2 * 2 + M * I * 2 * 2)

    def fused():
        return [thin_linear(thin_linear_silu_mul(x, gu[:I], gu[I:]), wd) for x, gu, wd in layers]

    def unfused():
        outs = []
        for x, gu, wd in layers:
            y = thin_linear(x, gu)
            outs.append(thin_linear(torch.nn.functional.silu(y[:, :I]) * y[:, I:], wd))
        return outs

    with torch.inference_mode():
        fused()
        unfused()
        torch.cuda.synchronize()
        us_unfused = graph_us_per_call(torch, [unfused], reps=max(5, args.steps // 5))
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fused()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fused()
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(args.steps):
            graph.replay()
        t1.record()
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / args.steps
    gbs = step_bytes / (ms * 1e-3) / 1e9
    return {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"gated-mlp-{L}L-H{H}-I{I}-M{M}", "M": M,
                   "algorithmic_bytes_per_step": step_bytes, "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "thin_linear_silu_mul + thin_linear (down), per layer"},
        "unfused_ms_per_step": round(us_unfused / 1e3, 4),
        "fused_speedup": round(us_unfused / 1e3 / ms, 3),
    }, M


# ───────────────────────────────────── decoder-layer linear path, fused ───
def run_layer(args, torch, dev):
    """Per layer: RMSNorm + qkv, o, RMSNorm + gate/up + SiLU-mul, down -- four
    launches with the norms and the gate epilogue fused (six above 8 tokens,
    where each norm is a launch of its own) -- against the
    unfused sequence (stock five-op RMSNorm in PyTorch, merged linears,
    PyTorch SiLU and product)."""
    from kernels.thin_linear_fused import (pick_config, thin_linear, thin_rmsnorm_linear,
                                           thin_rmsnorm_linear_silu_mul)

    M = int(args.workload[len("layer"):])
    if M == 4:
        H, QKV, I, L = 2048, 4096, 6144, 28
    else:
        H, QKV, I, L = 4096, 6144, 12288, 36
    # four launches, plus a norm launch for each of the two norms above 8
    # rows and a reduce launch for each split-K projection
    launches = 4 + (2 if M > 8 else 0) + sum(pick_config(M, N, K)[3] > 1
                                             for N, K in ((QKV, H), (H, H), (2 * I, H), (H, I)))
    eps = 1e-6
    layers = []
    for layer in range(L):
        g = torch.Generator(device=dev).manual_seed(6000 + layer)
        mk = lambda *sh, s=1.0: (torch.randn(*sh, device=dev, generator=g) * s).to(torch.bfloat16)
        layers.append(dict(x=mk(M, H), n1=(1 + 0.1 * torch.randn(H, device=dev, generator=g)).bfloat16(),
                           qkv=mk(QKV, H, s=0.02), o=mk(H, H, s=0.02), a=mk(M, H),
                           n2=(1 + 0.1 * torch.randn(H, device=dev, generator=g)).bfloat16(),
                           gu=mk(2 * I, H, s=0.02), down=mk(H, I, s=0.02)))
    wbytes = (QKV * H + H * H + 2 * I * H + H * I) * 2
    abytes = M * 2 * (H + QKV + H + H + H + H + I + I + H)
    step_bytes = L * (wbytes + abytes)

    def stock_norm(x, w):
        x32 = x.float()
        return w * (x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)

    def fused():
        out = []
        for d in layers:
            q = thin_rmsnorm_linear(d["x"], d["n1"], eps, d["qkv"])
            o = thin_linear(d["a"], d["o"])
            h = thin_rmsnorm_linear_silu_mul(d["x"], d["n2"], eps, d["gu"][:I], d["gu"][I:])
            out.append((q, o, thin_linear(h, d["down"])))
        return out

    def unfused():
        out = []
        for d in layers:
            q = thin_linear(stock_norm(d["x"], d["n1"]), d["qkv"])
            o = thin_linear(d["a"], d["o"])
            y = thin_linear(stock_norm(d["x"], d["n2"]), d["gu"])
            h = torch.nn.functional.silu(y[:, :I]) * y[:, I:]
            out.append((q, o, thin_linear(h, d["down"])))
        return out

    with torch.inference_mode():
        fused()
        unfused()
        torch.cuda.synchronize()
        us_unfused = graph_us_per_call(torch, [unfused], reps=max(5, args.steps // 5))
        us_fused = graph_us_per_call(torch, [fused], reps=args.steps)
    ms = us_fused / 1e3
    gbs = step_bytes / (ms * 1e-3) / 1e9
    return {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": 1, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"decoder-layer-linears-fused-{L}L-H{H}-M{M}", "M": M,
                   "launches_per_layer": launches, "algorithmic_bytes_per_step": step_bytes,
                   "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "RMSNorm+qkv, o, RMSNorm+gate/up+SiLU-mul, down per layer"},
        "unfused_ms_per_step": round(us_unfused / 1e3, 4),
        "fused_speedup": round(us_unfused / us_fused, 3),
    }, M


# ─────────────────────────────────────────────── lm_head + its epilogue ───
def run_head(args, torch, dev):
    """The lm_head and what follows it, fused against the reference's torch
    sequence.  head4: the draft's denoise step on a 4-token block (lm_head
    2048 -> 151936, softmax, argmax, confidence, masked top-1 unmasking with
    its step map and probability row; cache_aware.py:914-938).  head32: the
    target's verify pass over 32 rows (lm_head 4096 -> 151936, then softmax
    probabilities and argmax of the 16 mask rows; cache_aware.py:1197-1198)."""
    from kernels.logits_fused import denoise_select, softmax_argmax
    from kernels.thin_linear_fused import thin_linear
    F = torch.nn.functional

    M, K = (4, 2048) if args.workload == "head4" else (32, 4096)
    V = 151936
    mask_id = V - 1
    g = torch.Generator(device=dev).manual_seed(77)
    ws = [(torch.randn(V, K, device=dev, generator=g) * 0.02).to(torch.bfloat16) for _ in range(2)]
    xs = [torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16) for _ in range(2)]
    cur0 = torch.full((M,), mask_id, dtype=torch.int64, device=dev)
    cur = cur0.clone()
    step_map = torch.zeros(M, dtype=torch.int64, device=dev)
    ppp = torch.zeros(M, V, dtype=torch.float32, device=dev)
    lin_bytes = V * K * 2 + M * K * 2 + M * V * 2

    def fused():
        out = []
        for x, w in zip(xs, ws):
            if M == 4:
                cur.copy_(cur0)
                out.append(denoise_select(thin_linear(x, w), cur, mask_id, 1, 0, step_map, ppp))
            else:
                out.append(softmax_argmax(thin_linear(x, w)[16:32], return_probs=True))
        return out

    def unfused():
        out = []
        for x, w in zip(xs, ws):
            logits = thin_linear(x, w)
            if M == 4:
                cur.copy_(cur0)
                probs = F.softmax(logits.float(), dim=-1)
                pred = probs.argmax(dim=-1)
                conf = probs.gather(1, pred.unsqueeze(-1)).squeeze(-1)
                masked_conf = torch.where(cur == mask_id, conf, torch.full_like(conf, float("-inf")))
                _, top = masked_conf.topk(1)
                cur.scatter_(0, top, pred.gather(0, top))
                step_map.scatter_(0, top, torch.full_like(top, 0))
                ppp.index_copy_(0, top, probs.index_select(0, top))
                out.append((pred, conf))
            else:
                probs = F.softmax(logits[16:32].float(), dim=-1)
                out.append((probs.argmax(dim=-1), probs))
        return out

    with torch.inference_mode():
        fused()
        unfused()
        torch.cuda.synchronize()
        us_unfused = graph_us_per_call(torch, [unfused], reps=max(5, args.steps // 5)) / len(ws)
        us_fused = graph_us_per_call(torch, [fused], reps=args.steps) / len(ws)
        us_linear = graph_us_per_call(torch, [lambda x=x, w=w: thin_linear(x, w) for x, w in zip(xs, ws)],
                                      reps=args.steps)
    gbs = lin_bytes / (us_fused * 1e-6) / 1e9
    return {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": 1, "ms_per_step": round(us_fused / 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": ("draft-denoise-step-lm_head-M4-K2048-V151936" if M == 4 else
                                "target-verify-lm_head-M32-K4096-V151936-probs16"),
                   "M": M, "algorithmic_bytes_per_step": lin_bytes, "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "lm_head thin_linear + softmax/argmax epilogue (3 launches)"},
        "us_per_step": round(us_fused, 2),
        "lm_head_alone_us": round(us_linear, 2),
        "epilogue_us": round(us_fused - us_linear, 2),
        "unfused_us_per_step": round(us_unfused, 2),
        "unfused_epilogue_us": round(us_unfused - us_linear, 2),
        "fused_speedup": round(us_unfused / us_fused, 3),
    }, M


# ──────────────────────────────────────── attention over the static cache ───
def run_attn(args, torch, dev):
    """Per layer: q/k RMSNorm + RoPE + KV-cache write of the block's rows,
    then attention over a 1024-slot context: one launch
    (qkv_rope_attention) for the draft's 4 rows, two (qkv_rope_cache, then
    block_attention) for the target's 32.
    attn4: 28 draft layers, 4 rows, 16 query / 8 KV heads; attn32: 36 target
    layers, 32 rows (4 verify blocks), 32 / 8 heads.  The unfused timing is the
    reference's sequence (stock norms, apply_rotary_pos_emb, index_copy_ into
    the GQA-expanded cache, SDPA with the bool mask; SDPA pinned to its
    efficient kernel in bf16) on the same data."""
    from kernels.attention_fused import (BlockKVCache, block_attention, default_inv_freq, fused_attention_ok,
                                         gather_rope_rows, qkv_rope_attention, qkv_rope_cache, rope_table_pair,
                                         rope_tables)
    F = torch.nn.functional
    M, Hq, L_layers = (4, 16, 28) if args.workload == "attn4" else (32, 32, 36)
    Hkv, D, ctx, eps = 8, 128, args.context - M, 1e-6
    if ctx < 1 or args.context > 4096:
        raise SystemExit(f"bench.py: --context {args.context} must lie in ({M}, 4096]")
    n_rep = Hq // Hkv
    cache = BlockKVCache(L_layers, Hkv, ctx, M, dev)
    g = torch.Generator(device=dev).manual_seed(90)
    for lay in range(L_layers):
        cache.k_tiles[lay].normal_(generator=g)
        cache.v_tiles[lay].normal_(generator=g)
    cos, sin = rope_tables(default_inv_freq(device=dev), 4096, torch.bfloat16)
    qkvs = [torch.randn(M, (Hq + 2 * Hkv) * D, device=dev, generator=g).bfloat16() for _ in range(L_layers)]
    qn = (1 + 0.1 * torch.randn(D, device=dev, generator=g)).bfloat16()
    kn = (1 + 0.1 * torch.randn(D, device=dev, generator=g)).bfloat16()
    pos = torch.arange(ctx, ctx + M, device=dev)
    slots = torch.arange(cache.max_cache_len, cache.max_cache_len + M, device=dev)
    L = cache.max_cache_len + M
    mask = torch.zeros(M, cache.full_len, dtype=torch.bool, device=dev)
    mask[:, :ctx] = True
    mask[:, ctx:ctx + M] = torch.tril(torch.ones(M, M, dtype=torch.bool, device=dev))
    kv_bytes = Hkv * L * D * 2 * 2
    step_bytes = L_layers * (kv_bytes + M * (Hq + 2 * Hkv) * D * 2 + 2 * M * Hq * D * 2)

    one_launch = fused_attention_ok(M, Hq, Hkv, L)   # the rows sit at the last M valid slots

    pc, ps = rope_table_pair(cos, sin)

    def fused():
        if one_launch:   # as a decoder forward: the rows' cos / sin gathered once for every layer
            rows = gather_rope_rows(pc, ps, pos)
            return [qkv_rope_attention(x, Hq, qn, kn, eps, *rows, None, cache, lay, mask, valid_len=L)
                    for lay, x in enumerate(qkvs)]
        return [block_attention(qkv_rope_cache(x, Hq, qn, kn, eps, cos, sin, pos, slots, cache, lay),
                                cache, lay, mask, valid_len=L) for lay, x in enumerate(qkvs)]

    # the reference's expanded cache ([1, Hq, L, D]) holding the same context
    kexp = [cache.keys(lay).repeat_interleave(n_rep, 0)[None].contiguous() for lay in range(L_layers)]
    vexp = [cache.values(lay).repeat_interleave(n_rep, 0)[None].contiguous() for lay in range(L_layers)]
    c, s_ = cos[pos][:, None], sin[pos][:, None]

    def norm(t, w):
        t32 = t.float()
        return w * (t32 * torch.rsqrt(t32.pow(2).mean(-1, keepdim=True) + eps)).to(t.dtype)

    def rope(t):
        return (t * c) + (torch.cat((-t[..., 64:], t[..., :64]), dim=-1) * s_)

    def unfused():
        outs = []
        for lay, x in enumerate(qkvs):
            h = x.view(M, Hq + 2 * Hkv, D)
            q = rope(norm(h[:, :Hq], qn)).transpose(0, 1)[None]
            k = rope(norm(h[:, Hq:Hq + Hkv], kn)).transpose(0, 1)[None]
            v = h[:, Hq + Hkv:].transpose(0, 1)[None]
            for i in range(n_rep):
                kexp[lay][:, i::n_rep].index_copy_(2, slots, k)
                vexp[lay][:, i::n_rep].index_copy_(2, slots, v)
            o = F.scaled_dot_product_attention(q, kexp[lay], vexp[lay], attn_mask=mask[None, None],
                                               scale=D ** -0.5)
            outs.append(o.transpose(1, 2).reshape(M, Hq * D))
        return outs

    with torch.inference_mode():
        fused()
        torch.cuda.synchronize()
        us_fused = graph_us_per_call(torch, [fused], reps=args.steps)
        us_unfused, note = None, None
        try:
            from torch.nn.attention import SDPBackend, sdpa_kernel
            with sdpa_kernel([SDPBackend.EFFICIENT_ATTENTION]):
                unfused()
                torch.cuda.synchronize()
                us_unfused = graph_us_per_call(torch, [unfused], reps=max(5, args.steps // 5))
        except RuntimeError as e:   # no efficient bf16 kernel with a bool mask in this torch
            note = f"reference sequence not timed: {str(e).splitlines()[0][:160]}"
    ms = us_fused / 1e3
    gbs = step_bytes / (ms * 1e-3) / 1e9
    out = {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": 1, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"block-attention-{L_layers}L-M{M}-Hq{Hq}-Hkv{Hkv}-ctx{L}", "M": M,
                   "context_slots": L, "algorithmic_bytes_per_step": step_bytes, "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": ("qkv_rope_attention per layer (attn_head_rope_kernel: norm + RoPE + cache "
                                "write + attention in one launch; the rows' cos / sin gathered once for the "
                                "28 layers, counted in the time)" if one_launch else
                                "qkv_rope_cache + block attention per layer (attn_partial + attn_combine)")},
        "us_per_layer": round(us_fused / L_layers, 3),
        "unfused_us_per_layer": None if us_unfused is None else round(us_unfused / L_layers, 3),
        "fused_speedup": None if us_unfused is None else round(us_unfused / us_fused, 3),
    }
    if note:
        out["note"] = note
    return out, M


# ─────────────────────────────────────────────── the target's verify forward ───
def run_verify(args, torch, dev):
    """The SDAR-8B-shape target's verify forward at 36 rows over a 1024-slot
    context, one HIP graph per form: each projection's split-K partials handed
    to the launch that consumes them (reduce + q/k norm + RoPE + cache write,
    reduce + residual + RMSNorm), and the reduce-first form (a reduce launch,
    then the norm or the prologue).  Block-causal mask over the 36 rows (blocks
    of 4) after the context; lm_head on 16 of the rows."""
    from speculative.model import TARGET_8B, SynthModel

    M, ctx = 36, 1024 - 36
    model = SynthModel(TARGET_8B, dev, seed=12, max_ctx=1024, max_rows=64)
    full = model.cache.full_len
    g = torch.Generator(device=dev).manual_seed(5)
    for lay in range(TARGET_8B.n_layers):
        model.cache.k_tiles[lay].normal_(generator=g)
        model.cache.v_tiles[lay].normal_(generator=g)
    ids = torch.randint(0, TARGET_8B.vocab - 1, (M,), device=dev, generator=g)
    pos = torch.arange(ctx, ctx + M, device=dev)
    blk = torch.arange(M, device=dev) // 4
    mask = torch.zeros(M, full, dtype=torch.bool, device=dev)
    mask[:, :ctx] = True
    mask[:, ctx:ctx + M] = blk[None, :] <= blk[:, None]
    head_rows = torch.arange(4, M, 2, device=dev)[:16]

    def fwd():
        return model.forward(ids, pos, pos, mask, valid_len=ctx + M, head_rows=head_rows, rows_at_end=True)

    with torch.inference_mode():
        fwd()
        torch.cuda.synchronize()
        us_parts = graph_us_per_call(torch, [fwd], reps=args.steps)
        model.reduce_first = True
        fwd()
        torch.cuda.synchronize()
        us_first = graph_us_per_call(torch, [fwd], reps=args.steps)
        model.reduce_first = False
    sh = TARGET_8B
    H, D, I = sh.hidden, sh.head_dim, sh.intermediate
    layer_w = 2 * (H * (sh.n_q_heads + 2 * sh.n_kv_heads) * D + sh.n_q_heads * D * H + 2 * I * H + H * I)
    wbytes = sh.n_layers * layer_w + 2 * sh.vocab * H
    ms = us_parts / 1e3
    gbs = wbytes / (ms * 1e-3) / 1e9
    return {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": 1, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init weights)",
        "config": {"workload": "target-verify-forward-SDAR8B-36rows-ctx1024", "M": M, "context_slots": ctx + M,
                   "weight_bytes_per_step": wbytes, "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "whole forward: weight bytes / forward time"},
        "reduce_first_ms_per_step": round(us_first / 1e3, 4),
        "partials_speedup": round(us_first / us_parts, 3),
    }, M


# ───────────────────────────────────────────── end-to-end speculative step ───
def run_c5(args, torch, dev):
    """C5: random-init SDAR-1.7B draft and SDAR-8B target resident on one GPU,
    a 512-token prompt uniform over the vocabulary, 4-token blocks denoised in
    4 steps, K = 4 blocks verified per target forward (32 rows), greedy
    acceptance; the blocks an acceptance commits are folded into the next
    verify (their rows ahead of the 32, writing their K/V), so there is no
    separate extend forward.  value = generated tokens / second over the
    timed iterations.  The same run times, for comparison, the reference's
    separate extend forward on a second stream and in line, and the
    optimistic pipelined mode."""
    import time as _time

    from speculative.model import DRAFT_1P7B, TARGET_8B, SynthModel
    from speculative.step import SpecRunner

    steps, warm = args.steps, max(2, args.warmup)
    # every iteration commits at most K x 4 = 16 tokens: the timed ones, the
    # warmup, and three comparison modes of max(4, steps // 2) + 1 each
    max_ctx = 512 + 16 * (steps + warm + 3 * (max(4, steps // 2) + 1)) + 64
    t_init = _time.perf_counter()
    draft = SynthModel(DRAFT_1P7B, dev, seed=11, max_ctx=max_ctx, max_rows=64)
    target = SynthModel(TARGET_8B, dev, seed=12, max_ctx=max_ctx, max_rows=64)
    runner = SpecRunner(draft, target)
    prompt = torch.randint(0, DRAFT_1P7B.vocab - 1, (512,), generator=torch.Generator().manual_seed(5))
    runner.prefill(prompt)
    init_s = _time.perf_counter() - t_init
    for _ in range(warm):                 # captures the graphs
        runner.step()
    torch.cuda.synchronize()
    n_tok = n_acc = n_blocks = 0
    phase = [0.0, 0.0, 0.0, 0.0]
    t0 = _time.perf_counter()
    for _ in range(steps):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
        ctx0 = runner.ctx
        gen, acc = runner.step(events=ev[:4])
        ev[4].record()
        n_tok += len(gen)
        n_acc += acc
        n_blocks += (runner.ctx - ctx0) // runner.bl
        ev[4].synchronize()
        for i in range(4):
            phase[i] += ev[i].elapsed_time(ev[i + 1])
    runner.finish()
    torch.cuda.synchronize()
    secs = _time.perf_counter() - t0
    it_ms = secs * 1e3 / steps
    n_serial = max(4, steps // 2)

    def timed_mode(fold, overlap, pipelined):
        runner.fold, runner.overlap, runner.pipelined = fold, overlap, pipelined
        runner.step()                     # captures the mode's graphs (the first switch flushes)
        runner.finish()
        torch.cuda.synchronize()
        t = _time.perf_counter()
        for _ in range(n_serial):
            runner.step()
        runner.finish()
        torch.cuda.synchronize()
        return (_time.perf_counter() - t) * 1e3 / n_serial

    # the reference's separate extend forward, on a second stream beside the
    # next iteration's draft and in line; then the optimistic pipelined mode
    side_ms = timed_mode(False, True, False)
    serial_ms = timed_mode(False, False, False)
    pipe_ms = timed_mode(True, True, True)

    def layer_bytes(sh):
        H, D, I = sh.hidden, sh.head_dim, sh.intermediate
        return 2 * (H * (sh.n_q_heads + 2 * sh.n_kv_heads) * D + sh.n_q_heads * D * H + 2 * I * H + H * I)

    d_fwd = DRAFT_1P7B.n_layers * layer_bytes(DRAFT_1P7B) + 2 * DRAFT_1P7B.vocab * DRAFT_1P7B.hidden
    t_fwd = TARGET_8B.n_layers * layer_bytes(TARGET_8B)
    t_head = 2 * TARGET_8B.vocab * TARGET_8B.hidden
    d_fwds = runner.K * len(runner.schedule)
    # per iteration: the draft forwards and the verify (layers, with the
    # committed blocks folded in, and lm_head); a separate extend forward
    # would add t_fwd
    it_bytes = d_fwds * d_fwd + (t_fwd + t_head)
    gbs = it_bytes / (it_ms * 1e-3) / 1e9
    return {
        "metric": METRIC, "value": round(n_tok / secs, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": steps, "warmup": warm, "ms_per_step": round(it_ms, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init weights, uniform random prompt)",
        "config": {"workload": "spec-step-SDAR1.7B-draft-SDAR8B-target-bl4-ds4-K4-greedy-2stream",
                   "prompt": 512, "block_length": 4, "denoise_steps": 4, "k_blocks": 4,
                   "draft_forwards_per_iteration": d_fwds, "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "whole iteration: weight bytes of every forward / iteration time",
                     "bytes_per_iteration": int(it_bytes)},
        "tokens_per_iteration": round(n_tok / steps, 3),
        "accepted_draft_tokens_per_iteration": round(n_acc / steps, 3),
        "committed_blocks_per_iteration": round(n_blocks / steps, 3),
        "phase_ms_per_iteration": {"draft": round(phase[0] / steps, 3), "verify": round(phase[1] / steps, 3),
                                   "accept_host": round(phase[2] / steps, 3),
                                   "extend_issue": round(phase[3] / steps, 3)},
        "committed_blocks_folded_into_verify": True,
        "ms_per_iteration_extend_second_stream": round(side_ms, 3),
        "ms_per_iteration_extend_in_line": round(serial_ms, 3),
        "ms_per_iteration_pipelined": round(pipe_ms, 3),
        "pipelined_optimistic_drafts": dict(runner.stats),
        "hbm_bound_ms_per_iteration": round(it_bytes / 8e12 * 1e3, 3),
        "init_s": round(init_s, 1),
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline_c5(
            torch, (DRAFT_1P7B, TARGET_8B), d_fwds, 2, runner.ctx, n_tok / steps),
    }, 4


def cpu_baseline_c5(torch, shapes, d_fwds, t_fwds, ctx, tokens_per_iteration):
    """The reference's dense decoder forward in torch on the host cores
    (sdar/modeling_sdar.py: stock RMSNorm, F.linear q/k/v/o and gate/up/down,
    q/k RMSNorm, rotate-half RoPE, SDPA with a bool mask over a GQA-expanded
    cache of ``ctx`` slots, the static-cache path of adapters/base.py:186-265),
    bf16.  Bounded sample: one draft layer at 4 rows and one target layer at
    32 rows, each timed a few times, and both lm_heads once; the iteration is
    those times scaled by the iteration's forward counts (d_fwds draft
    forwards, t_fwds target forwards: the verify and the extend),
    tok/s = tokens per iteration / that."""
    F = torch.nn.functional
    g = torch.Generator().manual_seed(0)

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)

    def norm(t, w, eps):
        t32 = t.float()
        return w * (t32 * torch.rsqrt(t32.pow(2).mean(-1, keepdim=True) + eps)).to(t.dtype)

    def layer_fn(sh, M):
        H, D, Hq, Hkv, I = sh.hidden, sh.head_dim, sh.n_q_heads, sh.n_kv_heads, sh.intermediate
        w = {"ln1": 1 + rnd(H, scale=0.1), "wq": rnd(Hq * D, H, scale=0.02), "wk": rnd(Hkv * D, H, scale=0.02),
             "wv": rnd(Hkv * D, H, scale=0.02), "qn": 1 + rnd(D, scale=0.1), "kn": 1 + rnd(D, scale=0.1),
             "wo": rnd(H, Hq * D, scale=0.02), "ln2": 1 + rnd(H, scale=0.1), "wg": rnd(I, H, scale=0.02),
             "wu": rnd(I, H, scale=0.02), "wd": rnd(H, I, scale=0.02)}
        L = ctx + M
        kc, vc = rnd(1, Hq, L, D), rnd(1, Hq, L, D)          # the reference's expanded cache
        pos = torch.arange(ctx, ctx + M)
        inv = 1.0 / (sh.rope_theta ** (torch.arange(0, D, 2).float() / D))
        ang = torch.cat([pos[:, None].float() * inv[None]] * 2, dim=-1)
        cos, sin = ang.cos().to(torch.bfloat16)[:, None], ang.sin().to(torch.bfloat16)[:, None]
        mask = torch.ones(M, L, dtype=torch.bool)
        mask[:, ctx:] = torch.tril(torch.ones(M, M, dtype=torch.bool))
        x = rnd(M, H)
        slots = torch.arange(ctx, ctx + M)

        def rope(t):
            return t * cos + torch.cat((-t[..., D // 2:], t[..., :D // 2]), dim=-1) * sin

        def fwd():
            h = norm(x, w["ln1"], sh.eps)
            q = rope(norm(F.linear(h, w["wq"]).view(M, Hq, D), w["qn"], sh.eps))
            k = rope(norm(F.linear(h, w["wk"]).view(M, Hkv, D), w["kn"], sh.eps))
            v = F.linear(h, w["wv"]).view(M, Hkv, D)
            n_rep = Hq // Hkv
            kc.index_copy_(2, slots, k.repeat_interleave(n_rep, 1).transpose(0, 1)[None])
            vc.index_copy_(2, slots, v.repeat_interleave(n_rep, 1).transpose(0, 1)[None])
            a = F.scaled_dot_product_attention(q.transpose(0, 1)[None], kc, vc, attn_mask=mask[None, None])
            h2 = x + F.linear(a[0].transpose(0, 1).reshape(M, Hq * D), w["wo"])
            m = norm(h2, w["ln2"], sh.eps)
            return h2 + F.linear(F.silu(F.linear(m, w["wg"])) * F.linear(m, w["wu"]), w["wd"])
        return fwd

    def timed(fn, reps):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    draft, target = shapes
    with torch.inference_mode():
        t_d = timed(layer_fn(draft, 4), 5)
        t_t = timed(layer_fn(target, 32), 3)
        hd = (rnd(4, draft.hidden), rnd(draft.vocab, draft.hidden, scale=0.02))
        t_dh = timed(lambda: F.linear(*hd), 2)
        del hd
        ht = (rnd(32, target.hidden), rnd(target.vocab, target.hidden, scale=0.02))
        t_th = timed(lambda: F.linear(*ht), 2)
        del ht
    it_s = d_fwds * (draft.n_layers * t_d + t_dh) + t_fwds * target.n_layers * t_t + t_th
    return {
        "value": round(tokens_per_iteration / it_s, 4),
        "unit": "tok/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"reference decoder forward in torch on the host (bf16): one draft layer at 4 rows "
                   f"{t_d * 1e3:.2f} ms, one target layer at 32 rows {t_t * 1e3:.2f} ms, draft lm_head "
                   f"{t_dh * 1e3:.1f} ms, target lm_head {t_th * 1e3:.1f} ms (context {ctx} slots), scaled to "
                   f"{d_fwds} draft + {t_fwds} target forwards per iteration = {it_s * 1e3:.0f} ms for "
                   f"{tokens_per_iteration:.2f} tokens; cpu={cpu_model()}; os.cpu_count={os.cpu_count()}"),
    }


# ────────────────────────────────────────────────────────────────── MoE ───
def run_moe(args, torch, dev):
    from kernels.moe_dispatch_fused import moe_forward, moe_route

    T = int(args.workload[len("c4t"):])
    E, k, H, I, L = 256, 8, 2048, 512, 8
    layers = []
    for layer in range(L):
        g = torch.Generator(device=dev).manual_seed(300 + layer)
        mk = lambda *s: (torch.randn(*s, device=dev, generator=g) * 0.02).to(torch.bfloat16)
        logits = torch.randn(T, E, device=dev, generator=g)
        x = torch.randn(T, H, device=dev, generator=g).to(torch.bfloat16)
        layers.append((x, logits, mk(E, I, H), mk(E, I, H), mk(E, H, I), (mk(I, H), mk(I, H), mk(H, I))))
    per_expert = (2 * I * H + H * I) * BF16
    total_bytes = 0
    with torch.inference_mode():
        for x, logits, *_ in layers:
            ids, _ = moe_route(logits, k, scoring="softmax", renorm=False)
            n_active = int(torch.unique(ids).numel())
            total_bytes += (n_active + 1) * per_expert + T * H * BF16 * 2 + T * E * 4 + T * k * 12

    def step():
        return [moe_forward(x, lg, k, wg, wu, wd, shared=sh, scoring="softmax", renorm=False)
                for x, lg, wg, wu, wd, sh in layers]

    with torch.inference_mode():
        step()
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(args.steps):
            graph.replay()
        t1.record()
        torch.cuda.synchronize()
        ms_graph = t0.elapsed_time(t1) / args.steps
    ms = ms_graph / L
    gbs = total_bytes / L / (ms * 1e-3) / 1e9
    return {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps * L, "warmup": args.warmup * L, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"moe-step-T{T}-E{E}-k{k}-H{H}-I{I}+shared", "T": T,
                   "layers_cycled": L, "graph_replays": args.steps, "algorithmic_bytes_per_step": total_bytes // L,
                   "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(args.workload),
                     "kernel": "moe step (route+align, gate_up, down, combine; traffic per step)",
                     "bytes_per_step": total_bytes // L},
    }, T


def cpu_baseline_moe(torch, T):
    """The reference's CPU path for one MoE layer, in torch on the host cores
    in bf16: softmax top-8 routing, then the stock per-expert loop
    (kernels/workspace/moe_dispatch/build_oracle.py:34-67, the transcription
    of LLaDA2MoeSparseMoeBlock.moe_infer: histogram, argsort, one F.linear
    gate / up / SiLU.mul / down per active expert, scatter back, fp32
    weighting, sum) plus the shared expert.  Bounded sample: one stacked layer
    of all 256 experts (1.6 GB of bf16 weights, past any host cache) under 8
    distinct routings and inputs, cycled; GB/s over the same algorithmic
    bytes as the GPU step ((active experts + 1) x 6 MiB + activations)."""
    F = torch.nn.functional
    E, k, H, I, L = 256, 8, 2048, 512, 8
    g = torch.Generator().manual_seed(0)
    wg = torch.empty(E, I, H, dtype=torch.bfloat16)
    wu = torch.empty(E, I, H, dtype=torch.bfloat16)
    wd = torch.empty(E, H, I, dtype=torch.bfloat16)
    for t in (wg, wu, wd):                   # uniform, the spread of N(0, 0.02)
        t.uniform_(-0.0346, 0.0346, generator=g)
    shared = tuple((torch.randn(*s, generator=g) * 0.02).to(torch.bfloat16) for s in ((I, H), (I, H), (H, I)))
    layers = []
    per_expert = (2 * I * H + H * I) * BF16
    total_bytes = 0
    for _ in range(L):
        x = torch.randn(T, H, generator=g).to(torch.bfloat16)
        logits = torch.randn(T, E, generator=g)
        layers.append((x, logits))
        ids = torch.softmax(logits, dim=-1).topk(k, dim=-1).indices
        total_bytes += (int(torch.unique(ids).numel()) + 1) * per_expert + T * H * BF16 * 2 + T * E * 4 + T * k * 12

    def moe_layer(x, logits):
        w, ids = torch.softmax(logits, dim=-1).topk(k, dim=-1)
        cnts = ids.new_zeros((T, E))
        cnts.scatter_(1, ids, 1)
        tpe = cnts.sum(dim=0)
        idxs = ids.view(-1).argsort()
        sorted_tokens = x[idxs // k]
        outs, start = [], 0
        for e in range(E):
            n = int(tpe[e])
            if n == 0:
                continue
            toks = sorted_tokens[start:start + n]
            outs.append(F.linear(F.silu(F.linear(toks, wg[e])) * F.linear(toks, wu[e]), wd[e]))
            start += n
        o = torch.cat(outs)
        new_x = torch.empty_like(o)
        new_x[idxs] = o
        y = new_x.view(T, k, -1).to(w.dtype).mul_(w.unsqueeze(-1)).sum(1).to(new_x.dtype)
        sg, su, sd = shared
        return y + F.linear(F.silu(F.linear(x, sg)) * F.linear(x, su), sd)

    def step():
        for x, logits in layers:
            moe_layer(x, logits)

    with torch.inference_mode():
        step()                                 # warmup
        times = []
        t_end = time.perf_counter() + 12.0
        while len(times) < 20 and (time.perf_counter() < t_end or len(times) < 3):
            t0 = time.perf_counter()
            step()
            times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": round(total_bytes / med / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (f"torch CPU bf16: softmax top-{k} routing + the reference's stock per-expert loop "
                       f"(build_oracle.py:34-67) + the shared expert, T={T}, one 256-expert layer under "
                       f"{L} distinct routings cycled; median of {len(times)} passes "
                       f"({med * 1e3 / L:.2f} ms per layer); cpu={cpu_model()}; os.cpu_count={os.cpu_count()}")}


def run_copy(args, torch, dev):
    """A plain 1 GiB device copy (torch's elementwise copy kernel): the known
    byte count that calibrates the FETCH_SIZE / WRITE_SIZE counters."""
    n = 1 << 29   # bf16 elements = 1 GiB
    src = torch.empty(n, dtype=torch.bfloat16, device=dev).normal_()
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(args.steps):
        dst.copy_(src)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    byts = 2 * n * BF16
    return {"metric": "device copy GB/s (read + write)", "value": round(byts / (ms * 1e-3) / 1e9, 2),
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": 2,
            "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "copy-1GiB", "bytes_read": n * BF16, "bytes_written": n * BF16,
                       "parallelism": "single-gpu"}}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[1])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="c2",
                    choices=["c1", "c2", "c3m16", "c3m32", "c4t4", "c4t16", "c4t64", "mlp4", "mlp16",
                             "mlp32", "layer4", "layer16", "layer32", "layer36", "layer48", "head4", "head32",
                             "attn4", "attn32", "verify36", "c5", "copy"])
    ap.add_argument("--context", type=int, default=1024,
                    help="attn4 / attn32: valid cache slots once the new rows are written (default 1024)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="default workload only: skip the C1/C3/C4/C5 records that ride along")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: measures one MI355X; --gpus must be 1 (the hot path needs no "
              "communication between GPUs)",
              file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.workload == "copy":
        print(json.dumps(run_copy(args, torch, dev)), flush=True)
        return
    if args.workload == "c5":
        result, _ = run_c5(args, torch, dev)
        result["device"] = torch.cuda.get_device_name(dev)
        print(json.dumps(result), flush=True)
        return
    if args.workload.startswith(("mlp", "layer", "head", "attn", "verify")):
        runner = {"mlp": run_mlp, "layer": run_layer, "head": run_head,
                  "attn": run_attn, "verify": run_verify}[args.workload.rstrip("0123456789")]
        result, _ = runner(args, torch, dev)
        result["device"] = torch.cuda.get_device_name(dev)
        print(json.dumps(result), flush=True)
        return
    if args.workload.startswith("c4"):
        result, T = run_moe(args, torch, dev)
        if not args.no_cpu_baseline:
            result["cpu_baseline"] = cpu_baseline_moe(torch, T)
    else:
        result, M = run_linear(args, torch, dev)
        if not args.no_cpu_baseline:
            result["cpu_baseline"] = cpu_baseline_linear(torch, args.workload, M)
    result["device"] = torch.cuda.get_device_name(dev)
    if args.workload == "c2" and not args.no_extras:
        result["extras"] = run_extras(args, torch, dev)
    print(json.dumps(result), flush=True)


# The other configurations, timed in the same default run so that every
# number the metric names has a record from one invocation: C1 (the single
# gate_up), C3 at 16 and 32 rows, C4 at 4/16/64 tokens and C5 (the
# speculative step).  Each keeps its own algorithmic bytes, roofline fraction
# and per-op breakdown; the CPU baseline stays with the headline.
EXTRA_WORKLOADS = ("c1", "c3m16", "c3m32", "c4t4", "c4t16", "c4t64", "c5")
_EXTRA_KEYS = ("value", "unit", "ms_per_step", "steps", "config", "roofline", "breakdown", "tflops",
               "library_read_floor", "us_per_layer",
               "tokens_per_iteration", "accepted_draft_tokens_per_iteration", "committed_blocks_per_iteration",
               "phase_ms_per_iteration", "ms_per_iteration_extend_second_stream",
               "ms_per_iteration_extend_in_line", "ms_per_iteration_pipelined", "pipelined_optimistic_drafts",
               "hbm_bound_ms_per_iteration", "cpu_baseline")


def run_extras(args, torch, dev):
    """Each extra workload in a process of its own, one after another: in the
    process that has just run the C2 step, fresh allocations of the next
    workload's weights stream measurably slower (C1 10.8 against 10.0 us per
    call on one box), an effect of where the allocator places them, not of
    the kernels."""
    import subprocess

    out = {}
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    for wl in EXTRA_WORKLOADS:
        steps = 10 if wl == "c5" else max(10, args.steps // 2)
        warmup = 2 if wl == "c5" else max(2, args.warmup // 2)
        cmd = [sys.executable, os.path.abspath(__file__), "--workload", wl, "--steps", str(steps),
               "--warmup", str(warmup), "--no-extras"]
        # every extra carries its own host-core baseline (~10-20 s of CPU
        # work each, bounded inside the child)
        if args.no_cpu_baseline:
            cmd.append("--no-cpu-baseline")
        print(f"bench: extra workload {wl} ({steps} steps, own process)", file=sys.stderr, flush=True)
        t0 = time.perf_counter()
        # the child's progress goes straight to this process's stderr
        proc = subprocess.run(cmd, stdout=subprocess.PIPE, text=True, timeout=420)
        lines = [ln for ln in proc.stdout.splitlines() if ln.startswith("{")]
        if proc.returncode != 0 or not lines:
            raise RuntimeError(f"bench: extra workload {wl} failed (exit {proc.returncode})")
        rec = json.loads(lines[-1])
        rec = {k: rec[k] for k in _EXTRA_KEYS if k in rec}
        rec["wall_s"] = round(time.perf_counter() - t0, 1)
        out[wl] = rec
        print(f"bench: {wl} {rec['value']} {rec['unit']} in {rec['wall_s']} s", file=sys.stderr, flush=True)
    return out


if __name__ == "__main__":
    main()
