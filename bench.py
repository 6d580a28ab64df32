#!/usr/bin/env python3
"""Benchmark of the gfx950 weight-only qGEMM on one MI355X.

Workload (one "step"): the W4A16 decode sweep, group 128, fp16 activations,
(K, N) in {(5120, 5120), (5120, 27648), (27648, 5120)} x M in {1, 2, 4, 8, 16}:
15 GEMM launches. value = packed-weight + scale bytes of the whole step / step time
(GB/s). Weights rotate over >= 640 MiB of distinct copies per shape, so the 256 MiB
Infinity Cache cannot serve them. Steps are replayed as HIP graphs (one captured
graph per weight copy), which keeps host launch cost off the GPU timeline.

The same JSON line also carries:
  roofline      the dominant launch (K=5120, N=27648, M=16): algorithmic bytes (packed
                weights + scales) / average launch duration (HIP events around 64
                back-to-back launches on the launch stream), against 8 TB/s; `traffic`
                is the HBM bytes per launch from the committed rocprofv3 counter summary
                (profiles/decode_K5120_N27648_M16_traffic.json) when present;
  prefill       TFLOP/s of W4A16 M in {512, 2048, 4096}, K=5120, N=27648 and of the
                split-fuse mixed batch (fused QKV int4, fused gate||up ternary, M=1024),
                against the 2.5 PFLOP/s dense fp16 MFMA peak;
  cpu_baseline  the CPU oracle (restated reference dequantize-then-matmul, fp32) on the
                host cores over the same 15 GEMMs, repeated for about 10 s.

Usage:
  python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu] [--no-prefill]
  python bench.py --roofline-only        # the dominant launch only (for rocprofv3 --pmc)
  python bench.py --copy-bytes 268435456 # a plain device copy of known size (counter calibration)
  python bench.py --prefill-only 2048    # W4A16 prefill M=2048, K=5120, N=27648 only (for counters)
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
DOMINANT = (5120, 27648, 16)
TRAFFIC_FILE = ROOT / "profiles" / "decode_K5120_N27648_M16_traffic.json"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def wbytes(K: int, N: int, fmt: int = 1) -> int:
    """Algorithmic bytes of one launch: packed weights (int4 K*N/2, ternary K*N/4) + fp16 scales."""
    return (K * N // 2 if fmt == 1 else K * N // 4) + (K // GROUP) * N * 2


def make_weights(hq, torch, K, N, copies, fmt=1):
    """Distinct packed copies (device repack of random linear words) and |N(0, 0.02)| fp16 scales."""
    lin_words = hq.linear_words(fmt, K, N)
    ws, ss = [], []
    for _ in range(copies):
        if fmt == 1:
            lin = torch.randint(-2**31, 2**31 - 1, (lin_words,), dtype=torch.int32, device="cuda")
        else:  # ternary codes c = t + 1 with P(t) = (.25, .5, .25), 16 per word
            r = torch.randint(0, 4, (lin_words, 16), dtype=torch.int64, device="cuda")
            c = torch.where(r >= 2, 1, torch.where(r == 1, 2, 0))
            words = (c << (2 * torch.arange(16, device="cuda"))).sum(dim=1)
            lin = torch.where(words >= 2**31, words - 2**32, words).to(torch.int32)
        ws.append(hq.repack_device(fmt, lin, K, N))
        ss.append((torch.randn((K // GROUP, N), device="cuda").abs() * 0.02).to(torch.float16))
        del lin
    return ws, ss


def graph_time_us(torch, stream, launches, reps: int = 3) -> float:
    """Average duration of the launches captured in one HIP graph (events on the launch stream).
    One eager pass on the stream first, so that a shape needing the library's workspace gets
    it allocated outside the capture."""
    with torch.cuda.stream(stream):
        launches()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        n = launches()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        a.record(stream)
        for _ in range(reps):
            g.replay()
        b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / (reps * n)


def run_roofline_only(torch, hq):
    K, N, M = DOMINANT
    copies = max(2, -(-ROTATE_BYTES // wbytes(K, N)))
    ws, ss = make_weights(hq, torch, K, N, copies)
    X = torch.randn((M, K), device="cuda").to(torch.float16)
    Y = torch.empty((M, N), device="cuda", dtype=torch.float16)
    torch.cuda.synchronize()
    for r in range(4 * copies):
        hq.gemm(1, X, ws[r % copies], ss[r % copies], N, GROUP, out=Y)
    torch.cuda.synchronize()
    log(f"roofline-only: {4 * copies} launches of K={K} N={N} M={M}")


def run_prefill_only(torch, hq, M: int):
    K, N = 5120, 27648
    ws, ss = make_weights(hq, torch, K, N, 1)
    X = torch.randn((M, K), device="cuda").to(torch.float16)
    Y = torch.empty((M, N), device="cuda", dtype=torch.float16)
    for _ in range(5):
        hq.gemm(1, X, ws[0], ss[0], N, GROUP, out=Y)
    torch.cuda.synchronize()
    log(f"prefill-only: 5 launches of M={M} K={K} N={N}")


def run_copy(torch, nbytes: int):
    src = torch.empty(nbytes // 4, dtype=torch.int32, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy-only: 4 copies of {nbytes} bytes")


def traffic_from_profile():
    """HBM bytes per dominant launch from the committed counter summary, or None."""
    try:
        t = json.loads(TRAFFIC_FILE.read_text())
        f = t["fetch_kib"] * 1024 * t["copy_bytes"] / (t["copy_fetch_kib"] * 1024)
        w = t["write_kib"] * 1024 * t["copy_bytes"] / (t["copy_write_kib"] * 1024)
        return int(f + w)
    except (OSError, KeyError, ValueError, ZeroDivisionError):
        return None


def run_gpu(args):
    import torch

    from nebula_amd import hq

    dev = torch.cuda.get_device_properties(0)
    log(f"device {dev.name} CUs={dev.multi_processor_count} lib={hq.version()}")
    torch.manual_seed(0)
    stream = torch.cuda.Stream()

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

    with torch.cuda.stream(stream):
        step(0)  # eager pass before capture
    torch.cuda.synchronize()
    graphs = []
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
    with torch.cuda.stream(stream):
        e0.record(stream)
        for i in range(args.steps):
            graphs[i % R].replay()
        e1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"decode sweep: {ms_per_step * 1e3:.1f} us/step, {value:.1f} GB/s")

    # ---- per-case timing: 64 back-to-back launches over rotating weight copies ----
    cases = {}
    for K, N in SHAPES:
        ws, ss = pools[(K, N)]
        for M in MS:
            reps = len(ws) * max(1, 64 // len(ws))

            def launches(K=K, N=N, M=M, ws=ws, ss=ss, reps=reps):
                for r in range(reps):
                    hq.gemm(1, X[K][:M], ws[r % len(ws)], ss[r % len(ws)], N, GROUP, out=Y[(K, N)][:M])
                return reps

            us = graph_time_us(torch, stream, launches)
            gbs = wbytes(K, N) / (us * 1e-6) / 1e9
            cases[f"K{K}_N{N}_M{M}"] = {"us": round(us, 2), "GBps": round(gbs, 1),
                                        "pct_hbm": round(100 * gbs / HBM_PEAK_GBS, 1)}
    K, N, M = DOMINANT
    dom = cases[f"K{K}_N{N}_M{M}"]
    roofline = {"bound": "hbm", "achieved": dom["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(dom["GBps"] / HBM_PEAK_GBS, 4), "traffic": traffic_from_profile(),
                "kernel": f"hq_decode_ls_kernel<int4,f16,KG=2,T=2,U=2>, K={K} N={N} M={M}",
                "bytes_per_launch": wbytes(K, N), "avg_launch_us": dom["us"]}

    # ---- prefill and the split-fuse mixed batch ----
    prefill = None
    if not args.no_prefill:
        prefill = {}
        K, N = 5120, 27648
        ws, ss = pools[(K, N)]
        for M in (512, 2048, 4096):
            Xp = torch.randn((M, K), device="cuda").to(torch.float16)
            Yp = torch.empty((M, N), device="cuda", dtype=torch.float16)

            def launches(M=M, Xp=Xp, Yp=Yp):
                for r in range(len(ws)):
                    hq.gemm(1, Xp, ws[r], ss[r], N, GROUP, out=Yp)
                return len(ws)

            us = graph_time_us(torch, stream, launches, reps=2)
            tf = 2.0 * M * K * N / (us * 1e-6) / 1e12
            prefill[f"M{M}"] = {"us": round(us, 1), "TFLOPs": round(tf, 1),
                                "frac_mfma_f16": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}
            log(f"prefill M={M}: {us:.1f} us, {tf:.1f} TFLOP/s")
            del Xp, Yp
        # mixed split-fuse batch: 1008 prefill rows + 16 decode rows, fused QKV (int4) and gate||up (ternary)
        M = 1024
        Xm = torch.randn((M, 5120), device="cuda").to(torch.float16)
        qkv, gu = [], []
        for n in (5120, 1024, 1024):
            w, sc = make_weights(hq, torch, 5120, n, 1)
            qkv.append((w[0], sc[0], n))
        for n in (27648, 27648):
            w, sc = make_weights(hq, torch, 5120, n, 1, fmt=2)
            gu.append((w[0], sc[0], n))
        for name, fmt, seg_list in (("mixed_qkv_int4", 1, qkv), ("mixed_gate_up_ternary", 2, gu)):
            outs = [torch.empty((M, n), device="cuda", dtype=torch.float16) for (_, _, n) in seg_list]

            def launches(fmt=fmt, seg_list=seg_list, outs=outs):
                for _ in range(8):
                    hq.gemm_fused(fmt, Xm, seg_list, GROUP, outs=outs)
                return 8

            us = graph_time_us(torch, stream, launches, reps=2)
            ntot = sum(n for (_, _, n) in seg_list)
            tf = 2.0 * M * 5120 * ntot / (us * 1e-6) / 1e12
            prefill[name] = {"M": M, "N": ntot, "us": round(us, 1), "TFLOPs": round(tf, 1),
                             "frac_mfma_f16": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}
            log(f"{name}: {us:.1f} us, {tf:.1f} TFLOP/s")
    # ---- GGUF TQ1_0 import (model load): blocks -> packed ternary tiles + scales on the device ----
    K, N = 5120, 27648
    nbytes = hq.tq1_0_bytes(K, N)
    blocks = [torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda") for _ in range(4)]
    outs = hq.repack_tq1_0_device(blocks[0], K, N)

    def launches():
        for r in range(16):
            hq.repack_tq1_0_device(blocks[r % 4], K, N, out=outs)
        return 16

    us = graph_time_us(torch, stream, launches)
    moved = nbytes + 4 * hq.packed_words(hq.FORMAT_TERNARY2, K, N) + 2 * (K // 256) * N
    gbs = moved / (us * 1e-6) / 1e9
    tq1 = {"K": K, "N": N, "us": round(us, 1), "bytes": moved, "GBps": round(gbs, 1),
           "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
    log(f"TQ1_0 import K={K} N={N}: {us:.1f} us, {gbs:.1f} GB/s")
    del blocks, outs

    # ---- the reference decoder's layer projections (attention layer + FFN) as fused calls ----
    from nebula_amd import decoder as dec

    g = torch.Generator(device="cuda").manual_seed(11)
    layer = dec.random_layer("attention", generator=g)
    names = [n for grp in dec.FUSED_GROUPS["attention"] + dec.FUSED_GROUPS["ffn"] for n in grp]
    wbytes_layer = sum(hq.packed_words(hq.FORMAT_TERNARY2, *dec.SHAPES[n]) * 4 + (dec.SHAPES[n][0] // 256) *
                       dec.SHAPES[n][1] * 2 for n in names)
    flops_row = sum(2 * dec.SHAPES[n][0] * dec.SHAPES[n][1] for n in names)
    layer_res = {"weight_bytes": wbytes_layer}
    for M in (1, 16, 80, 512):
        xs = torch.randn((M, dec.EMBEDDING), device="cuda", generator=g).half()
        ys = torch.randn((M, dec.MIXER_IN), device="cuda", generator=g).half()
        acts = torch.randn((M, dec.FFN), device="cuda", generator=g).half()
        o_in = [torch.empty((M, dec.SHAPES[n][1]), device="cuda", dtype=torch.float16) for n in ("attn_q", "attn_k", "attn_v")]
        o_ffn = [torch.empty((M, dec.FFN), device="cuda", dtype=torch.float16) for _ in range(2)]
        o_x = torch.empty((M, dec.EMBEDDING), device="cuda", dtype=torch.float16)

        def launches(xs=xs, ys=ys, acts=acts, o_in=o_in, o_ffn=o_ffn, o_x=o_x):
            for _ in range(4):
                layer.mixer_in(xs, outs=o_in)
                layer.mixer_out(ys, out=o_x)
                layer.ffn_in(xs, outs=o_ffn)
                layer.ffn_out(acts, out=o_x)
            return 4

        us = graph_time_us(torch, stream, launches)
        layer_res[f"M{M}"] = {"us": round(us, 1), "GBps": round(wbytes_layer / (us * 1e-6) / 1e9, 1),
                              "TFLOPs": round(M * flops_row / (us * 1e-6) / 1e12, 1)}
        log(f"decoder layer projections M={M}: {us:.1f} us")
    # Token-by-token prefill (the reference runs prompt tokens one at a time) against one call.
    layer_res["prefill_512_speedup_vs_token_by_token"] = round(512 * layer_res["M1"]["us"] / layer_res["M512"]["us"], 1)
    del layer
    return value, ms_per_step, roofline, cases, prefill, tq1, layer_res


def run_cpu(budget_s: float = 10.0):
    """The CPU oracle (restated reference path) over the same 15 GEMMs, repeated for ~budget_s."""
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle as O

    threads = min(int(os.environ.get("OMP_NUM_THREADS", "0")) or min(16, os.cpu_count() or 1), 16)
    probs = {(K, N): O.Problem(O.INT4, 16, K, N, GROUP, O.F16, seed=7) for K, N in SHAPES}
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
    cpu = "host CPU"
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                cpu = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(done_bytes / t_used / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{sweeps} pass(es) over the 15 decode GEMMs (dequantize-then-matmul, fp32, "
                      f"{t_used:.1f} s) on {cpu}, {threads} threads of nproc={os.cpu_count()}"}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--roofline-only", action="store_true")
    ap.add_argument("--copy-bytes", type=int, default=0)
    ap.add_argument("--prefill-only", type=int, default=0)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): this qGEMM path runs on a single "
              "GPU and is not sharded here. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.roofline_only or args.copy_bytes or args.prefill_only:
        import torch

        from nebula_amd import hq

        if args.copy_bytes:
            run_copy(torch, args.copy_bytes)
        elif args.prefill_only:
            run_prefill_only(torch, hq, args.prefill_only)
        else:
            run_roofline_only(torch, hq)
        return
    value, ms_per_step, roofline, cases, prefill, tq1, layer_res = run_gpu(args)
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
        "tq1_0_import": tq1,
        "decoder_layer": layer_res,
        "cases": cases,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
