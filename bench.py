#!/usr/bin/env python3
"""Benchmark of the gfx950 weight-only qGEMM (one MI355X).

Workload (one "step"): the W4A16 decode sweep, group 128, fp16 activations,
(K, N) in {(5120, 5120), (5120, 27648), (27648, 5120)} x M in {1, 2, 4, 8, 16}:
15 GEMM launches. value = packed-weight + scale bytes of the whole step / step time
(GB/s); weights rotate over >= 512 MiB of distinct copies per shape so the 256 MiB
Infinity Cache cannot serve them. Steps are replayed as HIP graphs (one captured graph
per weight copy) so host launch cost stays off the GPU timeline.

Also reported, in the same JSON line:
  roofline     the dominant launch (K=5120, N=27648, M=16): algorithmic bytes / average
               launch duration from HIP events over back-to-back launches, vs 8 TB/s;
  prefill      W4A16 M=2048, K=5120, N=27648 TFLOP/s vs the 2.5 PFLOP/s fp16 MFMA peak;
  cpu_baseline the CPU oracle (restated reference dequantize-then-matmul) on the host
               cores over the same sweep (a bounded sample of about 10 s).

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu] [--no-prefill]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
SHAPES = [(5120, 5120), (5120, 27648), (27648, 5120)]
MS = [1, 2, 4, 8, 16]
GROUP = 128
ROTATE_BYTES = 640 << 20  # per shape, > 2x the 256 MiB MALL


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def wbytes(K: int, N: int) -> int:
    """Algorithmic bytes of one W4A16 launch: packed int4 weights + fp16 group scales."""
    return K * N // 2 + (K // GROUP) * N * 2


def make_weights(hq, torch, K, N, copies):
    """Distinct packed int4 copies (device repack of random linear words) and fp16 scales."""
    lin_words = hq.linear_words(1, K, N)
    ws, ss = [], []
    for _ in range(copies):
        lin = torch.randint(-2**31, 2**31 - 1, (lin_words,), dtype=torch.int32, device="cuda")
        ws.append(hq.repack_device(1, lin, K, N))
        ss.append((torch.randn((K // GROUP, N), device="cuda").abs() * 0.02).to(torch.float16))
        del lin
    return ws, ss


def run_gpu(args):
    import torch

    from nebula_amd import hq

    torch.cuda.init()
    dev = torch.cuda.get_device_properties(0)
    log(f"device {dev.name} CUs={dev.multi_processor_count} lib={hq.version()}")
    torch.manual_seed(0)

    # ---- decode sweep (the value) ----
    pools = {}
    for K, N in SHAPES:
        copies = max(2, -(-ROTATE_BYTES // wbytes(K, N)))
        pools[(K, N)] = make_weights(hq, torch, K, N, copies)
        log(f"shape K={K} N={N}: {copies} weight copies ({copies * wbytes(K, N) / 2**20:.0f} MiB)")
    X = {K: torch.randn((16, K), device="cuda").to(torch.float16) for K in {k for k, _ in SHAPES}}
    Y = {(K, N): torch.empty((16, N), device="cuda", dtype=torch.float16) for K, N in SHAPES}
    R = max(len(w) for w, _ in pools.values())
    step_bytes = sum(wbytes(K, N) for K, N in SHAPES for _ in MS)

    def step(i):
        for K, N in SHAPES:
            ws, ss = pools[(K, N)]
            c = i % len(ws)
            for M in MS:
                hq.gemm(1, X[K][:M], ws[c], ss[c], N, GROUP, out=Y[(K, N)][:M])

    stream = torch.cuda.Stream()
    graphs = []
    with torch.cuda.stream(stream):
        step(0)  # eager pass before capture
    torch.cuda.synchronize()
    for i in range(R):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            step(i)
        graphs.append(g)
    torch.cuda.synchronize()
    log(f"captured {R} step graphs of {len(SHAPES) * len(MS)} launches")

    for i in range(args.warmup):
        graphs[i % R].replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(args.steps):
        graphs[i % R].replay()
    e1.record()
    torch.cuda.synchronize()
    ms_total = e0.elapsed_time(e1)
    ms_per_step = ms_total / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"decode sweep: {ms_per_step * 1e3:.1f} us/step, {value:.1f} GB/s")

    # ---- per-case and dominant-launch timing (back-to-back graph of rotating launches) ----
    cases = {}
    for K, N in SHAPES:
        ws, ss = pools[(K, N)]
        for M in MS:
            reps = len(ws) * max(1, 64 // len(ws))
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for r in range(reps):
                    hq.gemm(1, X[K][:M], ws[r % len(ws)], ss[r % len(ws)], N, GROUP, out=Y[(K, N)][:M])
            g.replay()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(3):
                g.replay()
            b.record()
            torch.cuda.synchronize()
            us = a.elapsed_time(b) * 1e3 / (3 * reps)
            gbs = wbytes(K, N) / (us * 1e-6) / 1e9
            cases[f"K{K}_N{N}_M{M}"] = {"us": round(us, 2), "GBps": round(gbs, 1),
                                        "pct_hbm": round(100 * gbs / HBM_PEAK_GBS, 1)}
            del g
    dom = cases["K5120_N27648_M16"]
    roofline = {"bound": "hbm", "achieved": dom["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(dom["GBps"] / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": "hq_decode_kernel (int4, f16), K=5120 N=27648 M=16",
                "bytes_per_launch": wbytes(5120, 27648), "avg_launch_us": dom["us"]}

    # ---- prefill (config 3, M=2048) ----
    prefill = None
    if not args.no_prefill:
        K, N, M = 5120, 27648, 2048
        ws, ss = pools[(K, N)]
        Xp = torch.randn((M, K), device="cuda").to(torch.float16)
        Yp = torch.empty((M, N), device="cuda", dtype=torch.float16)
        hq.gemm(1, Xp, ws[0], ss[0], N, GROUP, out=Yp)
        torch.cuda.synchronize()
        reps = 4
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for r in range(reps):
            hq.gemm(1, Xp, ws[r % len(ws)], ss[r % len(ws)], N, GROUP, out=Yp)
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / reps
        tf = 2.0 * M * K * N / (us * 1e-6) / 1e12
        prefill = {"M": M, "K": K, "N": N, "us": round(us, 1), "TFLOPs": round(tf, 1),
                   "frac_mfma_f16": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}
        log(f"prefill M=2048: {us:.1f} us, {tf:.1f} TFLOP/s")
    return value, ms_per_step, roofline, cases, prefill


def run_cpu(budget_s: float = 10.0):
    """The CPU oracle over the same sweep, repeated until ~budget_s of work."""
    sys.path.insert(0, str(ROOT / "tests"))
    import numpy as np  # noqa: F401

    import oracle as O

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or min(16, os.cpu_count() or 1)
    threads = min(threads, 16)
    probs = {}
    for K, N in SHAPES:
        probs[(K, N)] = O.Problem(O.INT4, 16, K, N, GROUP, O.F16, seed=7)
    done_bytes, t_used, sweeps = 0, 0.0, 0
    while t_used < budget_s or sweeps == 0:
        for K, N in SHAPES:
            P = probs[(K, N)]
            for M in MS:
                t = time.perf_counter()
                O.qgemm(O.INT4, P.X[:M], O.F16, P.W, P.scales, N, GROUP, threads)
                t_used += time.perf_counter() - t
                done_bytes += wbytes(K, N)
        sweeps += 1
    gbs = done_bytes / t_used / 1e9
    cpu = ""
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                cpu = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{sweeps} full sweep(s) of the 15 decode GEMMs (dequantize-then-matmul, fp32, "
                      f"{t_used:.1f} s) on {cpu or 'host CPU'}, nproc={os.cpu_count()}"}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this path is not sharded. "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    value, ms_per_step, roofline, cases, prefill = run_gpu(args)
    cpu = None if args.no_cpu else run_cpu(args.cpu_budget)
    out = {
        "metric": "qGEMM GB/s at M<=16 (% of HBM peak) + TFLOP/s at M=2048 (% MFMA peak)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "W4A16 decode sweep, group 128, fp16 activations: (K,N) in "
                               "{(5120,5120),(5120,27648),(27648,5120)} x M in {1,2,4,8,16}",
                   "bytes_per_step": sum(wbytes(K, N) for K, N in SHAPES for _ in MS),
                   "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "prefill": prefill,
        "cases": cases,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
