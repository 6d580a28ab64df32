#!/usr/bin/env python3
"""Benchmark of the gfx950 weight-only qGEMM on one MI355X.

Workload (one "step"): the W4A16 decode sweep, group 128, fp16 activations,
(K, N) in {(5120, 5120), (5120, 27648), (27648, 5120)} x M in {1, 2, 4, 8, 16}:
15 GEMM launches. value = packed-weight + scale bytes of the whole step / step time
(GB/s). Every launch reads a weight copy that no launch of the previous ~640 MiB read
(copies rotate per launch over >= 640 MiB per shape), so the 256 MiB Infinity Cache cannot
serve them. Steps are replayed as HIP graphs, which keeps host launch cost off the GPU
timeline; inputs are resident in HBM before the timed region. After the warm-up steps,
untimed steps continue until 100 ms of them have run (the "settle" entry), whatever --warmup
is: the clock reaches its steady state only under lasting load (after 5 warm-up steps alone
the first timed steps ran up to 5% slower).

The same JSON line also carries:
  cases         per launch shape: average launch duration (HIP events on the launch stream
                around back-to-back launches of one captured graph, rotating weight copies),
                GB/s and fraction of the 8 TB/s HBM peak, and the plan (kernel, tiling) that
                ran. The decode sweep's 15 shapes, the single W4A16 GEMM (M=16, K=N=4096),
                the ternary bf16 decode (K=5120, N=27648, M in {1, 8}) and the int8 path
                (fp32 activations, int8 weights, K=5120, N=27648, M in {1, 8, 16}; bytes = int8
                weights + fp32 scales);
  roofline      the dominant decode kernel (the kernel with the largest share of the step
                time): its algorithmic bytes (packed weights + scales) per launch / its
                average launch duration, against 8 TB/s; `traffic` is the HBM bytes per
                launch measured in this run by two rocprofv3 --pmc passes (FETCH_SIZE,
                WRITE_SIZE) over that kernel's shape, each scaled by what the same counter
                reads for a plain device copy of known size (null if rocprofv3 is absent);
  prefill_M2048 the metric's second half: W4A16 M=2048, K=5120, N=27648 TFLOP/s against the
                2.5 PFLOP/s dense fp16 MFMA peak (also as roofline_prefill);
  prefill       M in {512, 2048, 4096} (each with hipBLASLt's dense fp16 GEMM on the same shape
                for reference) and the split-fuse mixed batch (fused QKV int4, fused
                gate||up ternary, M=1024);
  cpu_baseline  the CPU oracle (restated reference path: host dequantisation, then the fp32
                matmul) on the host cores over the 15 decode GEMMs: dequantisation and matmul
                timed separately, median of 5 runs each;
  stream_ceiling the practical read ceiling of each decode launch size on this device (the
                fastest plain streaming read of those bytes, nebula_amd/bin/hq_stream_ceiling,
                launch cost included) and the sweep's rate at that ceiling.

Usage:
  python bench.py [--gpus 1] [--steps 100] [--warmup 50] [--no-cpu] [--no-prefill] [--no-traffic] [--no-ceiling]
  (after the warm-up steps, untimed decode steps run until 100 ms have passed: the "settle"
  entry of the JSON line; the clock needs lasting load to reach its steady state)
  python bench.py --roofline-only --case K N M [--case-fmt ternary]  # one decode shape (rocprofv3 --pmc)
  python bench.py --copy-bytes 268435456        # a plain device copy of known size (counter calibration)
  python bench.py --prefill-only 2048           # W4A16 prefill M=2048, K=5120, N=27648 only (for counters)
  python bench.py --fused-only qkv|gateup       # the split-fuse batch's fused call at M=1024 only (for counters)
"""
from __future__ import annotations

import argparse
import csv
import json
import math
import os
import shutil
import statistics
import subprocess
import sys
import tempfile
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
SETTLE_MS = 100.0         # untimed decode steps run before the timed region, whatever --warmup is
BACKLOG = 10              # untimed steps queued right ahead of the timed region's start event
COPY_BYTES = 268435456    # counter calibration copy
FMT_INT4, FMT_TERN = 1, 2


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def wbytes(K: int, N: int, fmt: int = FMT_INT4) -> int:
    """Algorithmic bytes of one launch: packed weights (int4 K*N/2, ternary K*N/4) + fp16 scales."""
    return (K * N // 2 if fmt == FMT_INT4 else K * N // 4) + (K // GROUP) * N * 2


def n_copies(K: int, N: int, fmt: int = FMT_INT4) -> int:
    return max(2, -(-ROTATE_BYTES // wbytes(K, N, fmt)))


def make_weights(hq, torch, K, N, copies, fmt=FMT_INT4):
    """Distinct packed copies (device repack of random linear words) and |N(0, 0.02)| fp16 scales."""
    lin_words = hq.linear_words(fmt, K, N)
    ws, ss = [], []
    for _ in range(copies):
        if fmt == FMT_INT4:
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
        g.replay()  # queued ahead of the start event: the GPU is busy when the timing starts
        a.record(stream)
        for _ in range(reps):
            g.replay()
        b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / (reps * n)


def warm(torch, stream, launches, ms: float = 100.0) -> None:
    """Run `launches` eagerly on the stream for about `ms` milliseconds. A compute-bound launch
    timed right after other work runs up to 20% slower than the same launch under sustained
    load (measured on MI355X: prefill M=2048 526 us on the first graph, 438 us after 100 ms):
    the clock settles only after the load has lasted."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        e0.record(stream)
        n = launches()
        e1.record(stream)
    torch.cuda.synchronize()
    per = max(e0.elapsed_time(e1) / max(n, 1), 1e-3)
    with torch.cuda.stream(stream):
        for _ in range(int(ms / (per * max(n, 1))) + 1):
            launches()
    torch.cuda.synchronize()


def kernel_of(plan: str) -> str:
    """The kernel (template and parameters) of a plan description."""
    return plan.split(">", 1)[0] + ">"


# ---------------------------------------------------------------- single-purpose runs (profilers)
def run_case_only(torch, hq, K: int, N: int, M: int, ternary: bool = False):
    """One decode shape: int4 with fp16 activations, or ternary with bf16 ones."""
    fmt, dt, tdt = (FMT_TERN, 2, torch.bfloat16) if ternary else (FMT_INT4, 1, torch.float16)
    copies = n_copies(K, N, fmt)
    ws, ss = make_weights(hq, torch, K, N, copies, fmt)
    X = torch.randn((M, K), device="cuda").to(tdt)
    Y = torch.empty((M, N), device="cuda", dtype=tdt)
    torch.cuda.synchronize()
    for r in range(4 * copies):
        hq.gemm(fmt, X, ws[r % copies], ss[r % copies], N, GROUP, out=Y)
    torch.cuda.synchronize()
    log(f"case-only: {4 * copies} launches of K={K} N={N} M={M}: {hq.describe(fmt, dt, M, K, N)}")


def run_prefill_only(torch, hq, M: int):
    K, N = 5120, 27648
    ws, ss = make_weights(hq, torch, K, N, 1)
    X = torch.randn((M, K), device="cuda").to(torch.float16)
    Y = torch.empty((M, N), device="cuda", dtype=torch.float16)
    for _ in range(5):
        hq.gemm(FMT_INT4, X, ws[0], ss[0], N, GROUP, out=Y)
    torch.cuda.synchronize()
    log(f"prefill-only: 5 launches of M={M} K={K} N={N}")


def run_fused_only(torch, hq, which: str):
    """The split-fuse batch's fused call at M = 1024: QKV (int4, N = 5120 + 1024 + 1024) or
    gate||up (ternary, N = 2 x 27648), K = 5120, fp16 activations; 5 launches."""
    M, K = 1024, 5120
    fmt, ns = (FMT_INT4, (5120, 1024, 1024)) if which == "qkv" else (FMT_TERN, (27648, 27648))
    X = torch.randn((M, K), device="cuda").to(torch.float16)
    segs = []
    for n in ns:
        w, sc = make_weights(hq, torch, K, n, 1, fmt=fmt)
        segs.append((w[0], sc[0], n))
    outs = [torch.empty((M, n), device="cuda", dtype=torch.float16) for n in ns]
    for _ in range(5):
        hq.gemm_fused(fmt, X, segs, GROUP, outs=outs)
    torch.cuda.synchronize()
    log(f"fused-only: 5 launches of {which} M={M} K={K} N={'+'.join(map(str, ns))}")


def run_copy(torch, nbytes: int):
    src = torch.empty(nbytes // 4, dtype=torch.int32, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy-only: 4 copies of {nbytes} bytes")


# ---------------------------------------------------------------- HBM traffic (rocprofv3 --pmc)
def _pmc_pass(counter: str, args: list, outdir: str, tag: str):
    """One rocprofv3 counter pass over a child run of this script; per-dispatch values (KiB)."""
    cmd = ["timeout", "-s", "KILL", "120", "rocprofv3", "--pmc", counter, "-d", outdir, "-o", tag,
           "--output-format", "csv", "--", sys.executable, "-u", str(ROOT / "bench.py"), *args]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"{' '.join(cmd)} exited {p.returncode}: {p.stderr[-400:]}")
    rows = []
    for path in Path(outdir).rglob(f"{tag}_counter_collection.csv"):
        with open(path) as f:
            rows += [r for r in csv.DictReader(f) if r.get("Counter_Name") == counter]
    return rows


def measure_traffic(K: int, N: int, M: int, kernel: str):
    """HBM bytes per launch of the decode kernel at (K, N, M): FETCH_SIZE and WRITE_SIZE (KiB per
    dispatch) from two rocprofv3 --pmc passes, each scaled by bytes / counter of a plain copy of
    COPY_BYTES (FETCH_SIZE of a copy reads half its bytes on this part)."""
    if shutil.which("rocprofv3") is None:
        return None, "rocprofv3 not found"
    out = tempfile.mkdtemp(prefix="hq_pmc_")
    try:
        res = {}
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            dec = [float(r["Counter_Value"]) for r in
                   _pmc_pass(counter, ["--roofline-only", "--case", str(K), str(N), str(M)], out, "dec_" + counter)
                   if kernel.split("<")[0] in r["Kernel_Name"]]
            cpy = [float(r["Counter_Value"]) for r in
                   _pmc_pass(counter, ["--copy-bytes", str(COPY_BYTES)], out, "copy_" + counter)
                   if "copy" in r["Kernel_Name"].lower() or "elementwise" in r["Kernel_Name"].lower()]
            if not dec or not cpy:
                return None, f"{counter}: no dispatches matched ({len(dec)} kernel, {len(cpy)} copy)"
            res[counter] = (statistics.mean(dec), max(cpy), len(dec))
        f_kib, cf_kib, nd = res["FETCH_SIZE"]
        w_kib, cw_kib, _ = res["WRITE_SIZE"]
        traffic = f_kib * COPY_BYTES / cf_kib + w_kib * COPY_BYTES / cw_kib
        note = (f"FETCH_SIZE {f_kib:.1f} KiB x {COPY_BYTES / 1024 / cf_kib:.4f} + WRITE_SIZE {w_kib:.1f} KiB x "
                f"{COPY_BYTES / 1024 / cw_kib:.4f} per dispatch ({nd} dispatches); factors = copy bytes / counter "
                f"of a {COPY_BYTES}-byte device copy")
        return int(traffic), note
    except (RuntimeError, OSError, KeyError, ValueError) as e:
        return None, f"traffic not measured: {e}"
    finally:
        shutil.rmtree(out, ignore_errors=True)


# ---------------------------------------------------------------- stream ceiling
STREAM_TOOL = ROOT / "nebula_amd" / "bin" / "hq_stream_ceiling"


def case_bytes(key: str) -> int:
    """Algorithmic bytes of one launch of a decode case of the JSON line (0 for other cases)."""
    if key.startswith("K"):
        K, N = (int(x[1:]) for x in key.split("_")[:2])
        return wbytes(K, N)
    if key.startswith("single_"):
        return wbytes(4096, 4096)
    if key.startswith("ternary_"):
        K, N = (int(x[1:]) for x in key.split("_")[2:4])
        return wbytes(K, N, FMT_TERN)
    return 0


def stream_ceiling(value: float, cases=None):
    """The practical read ceiling of each decode launch size on this device, measured in this
    run by nebula_amd/bin/hq_stream_ceiling (the fastest of several launch shapes of a kernel
    that only reads the bytes once, HIP-graph timed over rotating buffers), the decode sweep's
    rate if every launch ran at that ceiling, and each decode case's time over its ceiling
    (the sweep's three sizes, the single 4096 x 4096 GEMM and the ternary launch)."""
    if not STREAM_TOOL.exists():
        return {"note": f"{STREAM_TOOL.relative_to(ROOT)} not built (run __graft_entry__.build())"}
    sizes = sorted({wbytes(K, N) for K, N in SHAPES} | {wbytes(4096, 4096), wbytes(5120, 27648, FMT_TERN)})
    p = subprocess.run(["timeout", "-k", "10", "120", str(STREAM_TOOL), *map(str, sizes)], capture_output=True, text=True)
    if p.returncode != 0:
        return {"note": f"hq_stream_ceiling exited {p.returncode}: {p.stderr[-300:]}"}
    res = json.loads(p.stdout)
    per = {str(s["bytes"]): {"us": round(s["us"], 3), "GBps": round(s["GBps"], 1),
                             "workgroups_per_cu": s["workgroups_per_cu"], "unroll": s["unroll"]} for s in res["sizes"]}
    step_us = sum(per[str(wbytes(K, N))]["us"] for K, N in SHAPES for _ in MS)
    step_bytes = sum(wbytes(K, N) for K, N in SHAPES for _ in MS)
    sweep = step_bytes / step_us / 1e3
    log(f"stream ceiling: {per}; sweep at the ceiling {sweep:.1f} GB/s ({100 * sweep / HBM_PEAK_GBS:.1f}% of peak)")
    over = {k: round(c["us"] / per[str(case_bytes(k))]["us"], 3) for k, c in (cases or {}).items()
            if str(case_bytes(k)) in per}
    return {"per_launch": per, "sweep_GBps": round(sweep, 1), "sweep_frac_hbm": round(sweep / HBM_PEAK_GBS, 3),
            "value_over_ceiling": round(value / sweep, 3), "case_over_ceiling": over,
            "note": "per decode launch size: the fastest plain read of those bytes (grid-stride 16-byte loads, "
                    "1-8 workgroups of 256 threads per CU, unroll 2-8), launch cost included"}


# ---------------------------------------------------------------- the GPU run
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
        pools[(K, N)] = make_weights(hq, torch, K, N, n_copies(K, N))
        log(f"shape K={K} N={N}: {len(pools[(K, N)][0])} weight copies "
            f"({len(pools[(K, N)][0]) * wbytes(K, N) / 2**20:.0f} MiB)")
    X = {K: torch.randn((16, K), device="cuda").to(torch.float16) for K in {k for k, _ in SHAPES}}
    Y = {(K, N): torch.empty((16, N), device="cuda", dtype=torch.float16) for K, N in SHAPES}
    step_bytes = sum(wbytes(K, N) for K, N in SHAPES for _ in MS)

    # Launch j of step i reads copy (i * len(MS) + j) mod copies: consecutive launches of a shape
    # never share a copy, and a copy comes back only after every other copy of the shape.
    def step(i):
        for K, N in SHAPES:
            ws, ss = pools[(K, N)]
            for j, M in enumerate(MS):
                c = (i * len(MS) + j) % len(ws)
                hq.gemm(FMT_INT4, X[K][:M], ws[c], ss[c], N, GROUP, out=Y[(K, N)][:M])

    R = 1
    for K, N in SHAPES:
        c = len(pools[(K, N)][0])
        R = R * (c // math.gcd(c, len(MS))) // math.gcd(R, c // math.gcd(c, len(MS)))
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
    # Settle: the clock reaches its steady state only after the load has lasted (after 5 warm-up
    # steps the first timed steps ran up to 5% slower), so untimed steps continue until SETTLE_MS
    # of them have run, whatever --warmup is; the JSON line reports how many. The copy rotation
    # continues across the warm-up, the settle and the timed steps.
    settle_steps, t0 = 0, time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < SETTLE_MS:
        for i in range(10):
            graphs[(args.warmup + settle_steps + i) % R].replay()
        settle_steps += 10
        torch.cuda.synchronize()
    settle_ms = (time.perf_counter() - t0) * 1e3
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        # A backlog of BACKLOG untimed steps queued ahead of the start event: a pause of the host
        # between two replays then never idles the GPU inside the timed region (with an empty
        # queue a 20-step region measured up to 25% slow on one box).
        for i in range(BACKLOG):
            graphs[(args.warmup + settle_steps + i) % R].replay()
        settle_steps += BACKLOG
        base = args.warmup + settle_steps
        e0.record(stream)
        for i in range(args.steps):
            graphs[(base + i) % R].replay()
        e1.record(stream)
    torch.cuda.synchronize()
    settle = {"ms": round(settle_ms, 1), "steps": settle_steps,
              "note": f"untimed decode steps after the {args.warmup} warm-up steps: until {SETTLE_MS:.0f} ms had run, "
                      f"then {BACKLOG} queued ahead of the timed region"}
    log(f"settle: {settle_steps} steps ({settle['ms']} ms, then {BACKLOG} queued)")
    ms_per_step = e0.elapsed_time(e1) / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"decode sweep: {ms_per_step * 1e3:.1f} us/step, {value:.1f} GB/s")
    del graphs

    # ---- per-case timing: back-to-back launches over rotating weight copies ----
    def time_case(fmt, K, N, M, ws, ss, Xk, Yk, dtype=1):
        reps = len(ws) * max(1, 64 // len(ws))

        def launches():
            for r in range(reps):
                hq.gemm(fmt, Xk[:M], ws[r % len(ws)], ss[r % len(ws)], N, GROUP, out=Yk[:M])
            return reps

        us = graph_time_us(torch, stream, launches)
        gbs = wbytes(K, N, fmt) / (us * 1e-6) / 1e9
        return {"us": round(us, 2), "GBps": round(gbs, 1), "pct_hbm": round(100 * gbs / HBM_PEAK_GBS, 1),
                "plan": hq.describe(fmt, dtype, M, K, N, GROUP)}

    cases = {}
    for K, N in SHAPES:
        ws, ss = pools[(K, N)]
        for M in MS:
            cases[f"K{K}_N{N}_M{M}"] = time_case(FMT_INT4, K, N, M, ws, ss, X[K], Y[(K, N)])
    # Dominant kernel: the largest share of the step's time (one launch per case and step).
    share = {}
    for key, c in cases.items():
        share.setdefault(kernel_of(c["plan"]), []).append(key)
    tot = sum(c["us"] for c in cases.values())
    dom_kernel = max(share, key=lambda k: sum(cases[c]["us"] for c in share[k]))
    dom_cases = share[dom_kernel]
    dom_us = sum(cases[c]["us"] for c in dom_cases)
    dom_bytes = sum(wbytes(int(c.split("_")[0][1:]), int(c.split("_")[1][1:])) for c in dom_cases)
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9
    # Its longest launch shape is the one the counter passes profile.
    prof_case = max(dom_cases, key=lambda c: cases[c]["us"])
    pK, pN, pM = (int(x[1:]) for x in prof_case.split("_"))
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel": dom_kernel,
                "launches": dom_cases, "share_of_step": round(dom_us / tot, 3),
                "bytes_per_launch": wbytes(pK, pN), "avg_launch_us": round(dom_us / len(dom_cases), 2),
                "traffic_case": prof_case}
    log(f"dominant kernel {dom_kernel}: {100 * dom_us / tot:.0f}% of the step, {achieved:.0f} GB/s")
    del pools, X, Y
    torch.cuda.empty_cache()

    # ---- the single W4A16 GEMM (M=16, K=N=4096) and the ternary bf16 decode ----
    K, N = 4096, 4096
    ws, ss = make_weights(hq, torch, K, N, n_copies(K, N))
    Xs, Ys = torch.randn((16, K), device="cuda").half(), torch.empty((16, N), device="cuda", dtype=torch.float16)
    cases["single_K4096_N4096_M16"] = time_case(FMT_INT4, K, N, 16, ws, ss, Xs, Ys)
    del ws, ss
    K, N = 5120, 27648
    ws, ss = make_weights(hq, torch, K, N, n_copies(K, N, FMT_TERN), fmt=FMT_TERN)
    Xt = torch.randn((8, K), device="cuda").to(torch.bfloat16)
    Yt = torch.empty((8, N), device="cuda", dtype=torch.bfloat16)
    for M in (1, 8):
        cases[f"ternary_bf16_K{K}_N{N}_M{M}"] = time_case(FMT_TERN, K, N, M, ws, ss, Xt, Yt, dtype=2)
    del ws, ss
    torch.cuda.empty_cache()

    # ---- the int8 path (forward_cutlass_int8's operands: fp32 activations, int8 [K][N] weights) ----
    K, N = 5120, 27648
    packed = torch.from_numpy(hq.repack_int8(torch.randint(-128, 128, (K, N), dtype=torch.int8).numpy()))
    copies = max(2, -(-ROTATE_BYTES // (K * N)))
    w8 = [packed.cuda() for _ in range(copies)]
    del packed
    s8 = torch.rand(N, device="cuda") * 0.1 + 0.05
    X8 = torch.randn((16, K), device="cuda") * 0.5
    Y8 = torch.empty((16, N), device="cuda")
    for M in (1, 8, 16):
        def launches(M=M):
            reps = copies * max(1, 64 // copies)
            for r in range(reps):
                hq.gemm_w8a8(X8[:M], w8[r % copies], s8, N, out=Y8[:M])
            return reps
        us = graph_time_us(torch, stream, launches)
        gbs = (K * N + N * 4) / (us * 1e-6) / 1e9
        cases[f"int8_w8a8_K{K}_N{N}_M{M}"] = {"us": round(us, 2), "GBps": round(gbs, 1),
                                             "pct_hbm": round(100 * gbs / HBM_PEAK_GBS, 1),
                                             "plan": "hq_gemm_w8a8: hq_w8a8_kernel, after hq_quantize_x_kernel "
                                                     "unless it quantises its own rows (one launch)"}
        log(f"int8 K={K} N={N} M={M}: {us:.2f} us, {gbs:.0f} GB/s")
    del w8
    torch.cuda.empty_cache()

    # ---- prefill and the split-fuse mixed batch ----
    prefill = None
    if not args.no_prefill:
        prefill = {}
        K, N = 5120, 27648
        ws, ss = make_weights(hq, torch, K, N, 3)
        for M in (512, 2048, 4096):
            Xp = torch.randn((M, K), device="cuda").to(torch.float16)
            Yp = torch.empty((M, N), device="cuda", dtype=torch.float16)

            def launches(M=M, Xp=Xp, Yp=Yp):
                for r in range(6):
                    hq.gemm(FMT_INT4, Xp, ws[r % 3], ss[r % 3], N, GROUP, out=Yp)
                return 6

            warm(torch, stream, launches)
            us = graph_time_us(torch, stream, launches, reps=3)
            tf = 2.0 * M * K * N / (us * 1e-6) / 1e12
            prefill[f"M{M}"] = {"us": round(us, 1), "TFLOPs": round(tf, 1),
                                "frac_mfma_f16": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                                "plan": hq.describe(FMT_INT4, 1, M, K, N, GROUP)}
            log(f"prefill M={M}: {us:.1f} us, {tf:.1f} TFLOP/s")
            # For reference, the vendor library on the same shape without quantisation: hipBLASLt's
            # dense fp16 GEMM through torch.matmul (weights [N][K], the layout it runs fastest).
            # Timed eagerly (back-to-back launches on one stream, HIP events), not captured, after
            # the same warm-up.
            Bt = torch.randn((N, K), device="cuda").to(torch.float16)

            def dense(Xp=Xp, Yp=Yp, Bt=Bt):
                for _ in range(6):
                    torch.matmul(Xp, Bt.t(), out=Yp)
                return 6

            warm(torch, stream, dense)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(stream):
                e0.record(stream)
                for _ in range(3):
                    dense()
                e1.record(stream)
            torch.cuda.synchronize()
            us_d = e0.elapsed_time(e1) * 1e3 / 18
            tf_d = 2.0 * M * K * N / (us_d * 1e-6) / 1e12
            prefill[f"M{M}"]["dense_fp16_hipblaslt"] = {"us": round(us_d, 1), "TFLOPs": round(tf_d, 1)}
            log(f"  dense fp16 (hipBLASLt) M={M}: {us_d:.1f} us, {tf_d:.1f} TFLOP/s")
            del Xp, Yp, Bt
        del ws, ss
        # mixed split-fuse batch: 1008 prefill rows + 16 decode rows, fused QKV (int4) and gate||up (ternary)
        M = 1024
        Xm = torch.randn((M, 5120), device="cuda").to(torch.float16)
        qkv, gu = [], []
        for n in (5120, 1024, 1024):
            w, sc = make_weights(hq, torch, 5120, n, 1)
            qkv.append((w[0], sc[0], n))
        for n in (27648, 27648):
            w, sc = make_weights(hq, torch, 5120, n, 1, fmt=FMT_TERN)
            gu.append((w[0], sc[0], n))
        for name, fmt, seg_list in (("mixed_qkv_int4", FMT_INT4, qkv), ("mixed_gate_up_ternary", FMT_TERN, gu)):
            outs = [torch.empty((M, n), device="cuda", dtype=torch.float16) for (_, _, n) in seg_list]

            def launches(fmt=fmt, seg_list=seg_list, outs=outs):
                for _ in range(8):
                    hq.gemm_fused(fmt, Xm, seg_list, GROUP, outs=outs)
                return 8

            warm(torch, stream, launches)
            us = graph_time_us(torch, stream, launches, reps=3)
            ntot = sum(n for (_, _, n) in seg_list)
            tf = 2.0 * M * 5120 * ntot / (us * 1e-6) / 1e12
            prefill[name] = {"M": M, "N": ntot, "us": round(us, 1), "TFLOPs": round(tf, 1),
                             "frac_mfma_f16": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}
            log(f"{name}: {us:.1f} us, {tf:.1f} TFLOP/s")
        del Xm, qkv, gu
        torch.cuda.empty_cache()

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
    return value, ms_per_step, settle, roofline, cases, prefill, tq1, layer_res


# ---------------------------------------------------------------- CPU baseline
def cpu_model() -> str:
    fields = {}
    try:
        for ln in open("/proc/cpuinfo"):
            k, _, v = ln.partition(":")
            k = k.strip()
            if k in ("model name", "cpu family", "model", "stepping") and k not in fields:
                fields[k] = v.strip()
    except OSError:
        pass
    name = fields.get("model name", "host CPU")
    ident = ", ".join(f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields)
    return f"{name} ({ident})" if ident else name


def run_cpu(reps: int = 5):
    """The CPU oracle (restated reference path) over the 15 decode GEMMs: per shape the host
    dequantisation (marlin_gemm.cu:495-512) once, then the fp32 matmul (:60-69) per M; each timed
    `reps` times, medians summed."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "tests"))
    import oracle as O

    threads = min(int(os.environ.get("OMP_NUM_THREADS", "0")) or min(16, os.cpu_count() or 1), 16)
    os.environ["OMP_NUM_THREADS"] = str(threads)
    dq_ms, mm_ms, total_s = {}, {}, 0.0
    for K, N in SHAPES:
        P = O.Problem(O.INT4, 16, K, N, GROUP, O.F16, seed=7)
        Xf = O.to_f32(P.X, O.F16)
        W = np.empty((K, N), dtype=np.float32)  # the reference's W_dequant buffer, allocated once
        W.fill(1.0)  # touched, so that no timed run pays its page faults
        t_dq = []
        for _ in range(reps):
            t = time.perf_counter()
            O.dequant(O.INT4, P.W, P.scales.ravel(), K, N, GROUP, out=W)
            t_dq.append(time.perf_counter() - t)
        dq_ms[f"K{K}_N{N}"] = round(1e3 * statistics.median(t_dq), 2)
        for M in MS:
            t_mm = []
            for _ in range(reps):
                t = time.perf_counter()
                O.gemm_f32(np.ascontiguousarray(Xf[:M]), W, threads)
                t_mm.append(time.perf_counter() - t)
            mm_ms[f"K{K}_N{N}_M{M}"] = round(1e3 * statistics.median(t_mm), 2)
            total_s += sum(t_mm)
        total_s += sum(t_dq)
        del W
    sweep_s = (sum(dq_ms.values()) + sum(mm_ms.values())) / 1e3
    step_bytes = sum(wbytes(K, N) for K, N in SHAPES for _ in MS)
    return {"value": round(step_bytes / sweep_s / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": (f"the 15 decode GEMMs once each: per shape the host dequantisation, then the fp32 matmul "
                       f"per M, each the median of {reps} runs ({total_s:.1f} s of CPU work) on {cpu_model()}, "
                       f"{threads} OpenMP threads of nproc={os.cpu_count()}"),
            "ms_per_sweep": round(1e3 * sweep_s, 1), "dequant_ms": dq_ms, "matmul_ms": mm_ms}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-traffic", action="store_true")
    ap.add_argument("--no-ceiling", action="store_true")
    ap.add_argument("--cpu-reps", type=int, default=5)
    ap.add_argument("--roofline-only", action="store_true")
    ap.add_argument("--case", type=int, nargs=3, default=[5120, 27648, 16], metavar=("K", "N", "M"))
    ap.add_argument("--case-fmt", choices=["int4", "ternary"], default="int4",
                    help="--roofline-only: int4 weights with fp16 activations, or ternary with bf16 ones")
    ap.add_argument("--copy-bytes", type=int, default=0)
    ap.add_argument("--prefill-only", type=int, default=0)
    ap.add_argument("--fused-only", choices=["qkv", "gateup"], default=None)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): this qGEMM path runs on a single "
              "GPU and is not sharded here. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.roofline_only or args.copy_bytes or args.prefill_only or args.fused_only:
        import torch

        from nebula_amd import hq

        if args.copy_bytes:
            run_copy(torch, args.copy_bytes)
        elif args.prefill_only:
            run_prefill_only(torch, hq, args.prefill_only)
        elif args.fused_only:
            run_fused_only(torch, hq, args.fused_only)
        else:
            run_case_only(torch, hq, *args.case, ternary=args.case_fmt == "ternary")
        return
    value, ms_per_step, settle, roofline, cases, prefill, tq1, layer_res = run_gpu(args)
    ceiling = None if args.no_ceiling else stream_ceiling(value, cases)
    if not args.no_traffic:
        K, N, M = (int(x[1:]) for x in roofline["traffic_case"].split("_"))
        roofline["traffic"], roofline["traffic_note"] = measure_traffic(K, N, M, roofline["kernel"])
        log(f"traffic of {roofline['kernel']} at K={K} N={N} M={M}: {roofline['traffic']} ({roofline['traffic_note']})")
    cpu = None if args.no_cpu else run_cpu(args.cpu_reps)
    out = {
        "metric": "qGEMM GB/s at M<=16 (% of HBM peak) + TFLOP/s at M=2048 (% MFMA peak)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": settle,
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
        "stream_ceiling": ceiling,
    }
    if prefill:
        p = prefill["M2048"]
        out["prefill_M2048"] = {"TFLOPs": p["TFLOPs"], "frac_mfma_f16": p["frac_mfma_f16"], "us": p["us"],
                                "workload": "W4A16 prefill M=2048 K=5120 N=27648 group 128 fp16"}
        out["roofline_prefill"] = {"bound": "mfma", "achieved": p["TFLOPs"], "peak": MFMA_F16_PEAK_TFLOPS,
                                   "unit": "TFLOP/s", "frac": p["frac_mfma_f16"], "traffic": None,
                                   "kernel": kernel_of(p["plan"]), "flops_per_launch": 2 * 2048 * 5120 * 27648,
                                   "avg_launch_us": p["us"]}
    out.update({"prefill": prefill, "tq1_0_import": tq1, "decoder_layer": layer_res, "cases": cases})
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
