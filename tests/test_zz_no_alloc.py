"""GPU test of hq_gemm_fused_noalloc, the entry point that allocates nothing (its workspace is
the library's static per-GPU scratch array), called through the C ABI and checked against
hq_gemm_fused on the same inputs: two calls in a row per case, the second with a smaller input.
The scratch keeps the first call's contents; a call that found its arrival counters not back at
zero would combine the wrong partial tiles, so the second call of each pair (and every later
case, all on the same scratch) also checks that the first left them at zero.

Cases whose plans need a workspace (each plan asserted through hq.describe):
  * the lockstep decode kernel with slabs cut along K (K=27648, N=5120, M=16), then the
    X-resident kernel in three K pieces (same shape, M=8);
  * the X-resident kernel in three K pieces (M=4), then whole slabs (M=1, no workspace);
  * the per-wavefront decode kernel (HQ_DECODE_KERNEL=0) with slabs cut by its workgroup
    ranges and their fix-up (M=4, then M=1);
  * the lockstep kernel's balanced grid (int4 5120 x 34816, M=32: 272 slabs on 256
    workgroups, first and last slabs shared through the scratch), then M=24;
  * prefill stream-K (M=100, K=4096, N=1024: 64-row tiles split along K; then M=90, N=512);
  * a prefill call whose usual stream-K workspace is larger than the scratch (M=1024,
    K=27648, N=5120): the no-allocation plan runs whole tiles instead, so the outputs agree up
    to fp32 summation order.
Bar: the same plan gives the same bits; a different plan agrees within the output-rounding
bound (normwise 2e-3 for fp16), and both meet the 1e-2 bar against the CPU oracle on rows.
"""
import os

import numpy as np
import pytest

import oracle as O
from gpu_util import to_dev_u16, to_dev_u32, to_host_f32
from nebula_amd import hq

pytestmark = pytest.mark.gpu


def problem(M, K, Ns, seed):
    probs = [O.Problem(O.INT4, M, K, n, 128, O.F16, seed=seed + i) for i, n in enumerate(Ns)]
    for p in probs[1:]:
        p.X = probs[0].X
    segs = [(to_dev_u32(hq.repack(O.INT4, p.W, K, p.N)), to_dev_u16(p.scales), p.N) for p in probs]
    return probs, to_dev_u16(probs[0].X, O.F16), segs


def run_pair(M, K, Ns, seed, same_plan=True, rows=None, plan=None):
    import torch

    if plan is not None:
        desc = hq.describe(O.INT4, O.F16, M, K, sum(Ns))
        assert plan in desc, (plan, desc)
    probs, X, segs = problem(M, K, Ns, seed)
    ref = hq.gemm_fused(O.INT4, X, segs)
    outs = [torch.full((M, n), 7.0, dtype=torch.float16, device="cuda") for n in Ns]
    hq.gemm_fused(O.INT4, X, segs, outs=outs, noalloc=True)
    torch.cuda.synchronize()
    hq.device_status()
    for p, a, b in zip(probs, outs, ref):
        if same_plan:
            assert bool(torch.equal(a, b)), f"M={M} K={K} N={p.N}: not bit-identical"
        ya, yb = to_host_f32(a), to_host_f32(b)
        assert O.normwise_error(ya, yb) <= 2e-3
        r = rows if rows is not None else np.arange(M)
        assert O.normwise_error(ya[r], p.reference(rows=r, threads=16)) <= 2e-3


@pytest.mark.parametrize("first,second", [((16, 27648, [5120], "hq_decode_ls_kernel<"), (8, 27648, [5120], "x 3 pieces")),
                                          ((4, 27648, [5120], "x 3 pieces"), (1, 27648, [5120], "x 1 pieces")),
                                          ((100, 4096, [1024], "whole=0 stream-K"), (90, 4096, [512], "whole=0 stream-K"))])
def test_noalloc_equals_fused_twice(cuda, first, second):
    for i, (M, K, Ns, plan) in enumerate((first, second)):
        run_pair(M, K, Ns, 7000 + 10 * i, plan=plan)


def test_noalloc_per_wavefront_kernel_cut_slabs(cuda):
    old = os.environ.get("HQ_DECODE_KERNEL")
    os.environ["HQ_DECODE_KERNEL"] = "0"
    try:
        for i, M in enumerate((4, 1)):
            run_pair(M, 27648, [5120], 7050 + 10 * i, plan="cut slabs (fix-up)")
    finally:
        if old is None:
            os.environ.pop("HQ_DECODE_KERNEL", None)
        else:
            os.environ["HQ_DECODE_KERNEL"] = old


def test_noalloc_balanced_grid(cuda):
    rows = np.array([0, 7, 16, 31])
    for i, M in enumerate((32, 24)):
        run_pair(M, 5120, [34816], 7070 + 10 * i, rows=rows[rows < M], plan="balanced grid")


def test_noalloc_plan_under_the_scratch_cap(cuda):
    # The usual plan's stream-K workspace exceeds the scratch: whole tiles instead.
    need = hq.workspace_bytes_fused(O.INT4, 1024, 27648, [5120])
    assert need > hq.NOALLOC_SCRATCH_BYTES
    rows = np.sort(np.random.default_rng(3).choice(1024, 12, replace=False))
    run_pair(1024, 27648, [5120], 7100, same_plan=False, rows=rows)
    run_pair(300, 27648, [2560], 7110, same_plan=False, rows=rows[rows < 300])


def test_noalloc_fused_segments(cuda):
    # QKV-shaped fused call at decode and split-fuse sizes.
    run_pair(16, 5120, [5120, 1024, 1024], 7200)
    run_pair(80, 5120, [5120, 1024, 1024], 7210)
