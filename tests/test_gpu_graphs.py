"""GPU test of the qGEMM under HIP graph capture: one call captured (through the C ABI, on a
capture stream of default priority, outputs and workspace allocated beforehand), the graph
replayed several times with eager calls of the same shape and synchronisations between the
replays, and every replay compared bit for bit with the eager result of the same plan.

The plans that meet through a workspace (X-resident K pieces, the lockstep kernel's K pieces and
balanced grid, prefill stream-K) must leave their arrival counters at zero after every launch,
since a graph replays the same launch over the same workspace with nothing in between; the
entry point that allocates nothing is captured as well (its workspace is the library's static
scratch). The launches record no memory set: the counters are left at zero by the kernels.
"""
import pytest

import oracle as O
from gpu_util import DeviceProblem
from nebula_amd import hq

pytestmark = pytest.mark.gpu

# (label, format, activation dtype, M, K, N, expected plan fragment)
CASES = [
    ("slab pairs", O.INT4, O.F16, 8, 5120, 27648, ",SG=2>"),
    ("X-resident K pieces", O.INT4, O.F16, 4, 27648, 5120, "x 3 pieces"),
    ("lockstep K pieces", O.INT4, O.F16, 16, 27648, 5120, "hq_decode_ls_kernel<int4,f16,KG=4"),
    ("lockstep balanced grid", O.INT4, O.F16, 32, 5120, 34816, "balanced grid"),
    ("ternary X-resident", O.TERNARY2, O.BF16, 1, 5120, 27648, "hq_decode_xr_kernel<ternary2,bf16"),
    ("prefill stream-K", O.INT4, O.F16, 100, 4096, 1024, "whole=0 stream-K"),
]


def capture(fn, side):
    import torch

    g = torch.cuda.CUDAGraph()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g, stream=side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    return g


@pytest.mark.parametrize("label,fmt,xdt,M,K,N,plan", CASES, ids=[c[0] for c in CASES])
def test_graph_replays_equal_eager(cuda, label, fmt, xdt, M, K, N, plan):
    import torch

    desc = hq.describe(fmt, xdt, M, K, N)
    assert plan in desc, (label, desc)
    P = O.Problem(fmt, M, K, N, 128, xdt, seed=9900 + M)
    D = DeviceProblem(P)
    need = hq.workspace_bytes(fmt, M, K, N)
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device="cuda") if need else None
    gemm = lambda out: hq.gemm(fmt, D.X, D.Wp, D.S, N, 128, out=out, workspace=ws)
    y0 = gemm(None)
    torch.cuda.synchronize()
    out = torch.empty_like(y0)
    g = capture(lambda: gemm(out), torch.cuda.Stream())
    for r in range(4):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert bool(torch.equal(out, y0)), f"{label}: replay {r} differs from the eager result ({desc})"
        y1 = gemm(None)  # an eager call over the same workspace between replays
        torch.cuda.synchronize()
        assert bool(torch.equal(y1, y0)), f"{label}: eager call after replay {r} differs ({desc})"


def test_graph_replays_noalloc_fused(cuda):
    # The entry point that allocates nothing, captured: 27648 x 5120 at M = 16 (the lockstep
    # kernel's K pieces through the static scratch) in one fused call of two segments.
    import torch

    M, K, Ns = 16, 27648, [5120, 1024]
    probs = [O.Problem(O.INT4, M, K, n, 128, O.F16, seed=9950 + i) for i, n in enumerate(Ns)]
    for p in probs[1:]:
        p.X = probs[0].X
    devs = [DeviceProblem(p) for p in probs]
    segs = [(d.Wp, d.S, d.P.N) for d in devs]
    ref = hq.gemm_fused(O.INT4, devs[0].X, segs, noalloc=False)
    outs = [torch.empty((M, n), dtype=torch.float16, device="cuda") for n in Ns]
    hq.gemm_fused(O.INT4, devs[0].X, segs, outs=outs, noalloc=True)
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    for a, b in zip(eager, ref):
        assert bool(torch.equal(a, b))
    g = capture(lambda: hq.gemm_fused(O.INT4, devs[0].X, segs, outs=outs, noalloc=True), torch.cuda.Stream())
    for r in range(4):
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert bool(torch.equal(o, e)), f"noalloc replay {r}, segment {i} differs from the eager result"
        hq.gemm_fused(O.INT4, devs[0].X, segs, outs=[torch.empty_like(o) for o in outs], noalloc=True)
        torch.cuda.synchronize()
    hq.device_status()
