"""GPU test of hq_gemm_fused_noalloc, the entry point that allocates nothing (its workspace is
the library's static per-GPU scratch array), called through the C ABI and checked against
hq_gemm_fused on the same inputs: two calls in a row per case, the second with a smaller input
(the scratch keeps the first call's contents, its arrival counters must be back at zero).

Cases whose plans need a workspace:
  * the lockstep decode kernel with slabs cut along K (K=27648, N=5120, M=16 then M=8);
  * the per-wavefront decode kernel with cut slabs and its fix-up (same shape, M=4 then M=1);
  * prefill stream-K (M=100, K=4096, N=1024: 64-row tiles split along K; then M=90, N=512);
  * a prefill call whose usual stream-K workspace is larger than the scratch (M=1024,
    K=27648, N=5120): the no-allocation plan runs whole tiles instead, so the outputs agree up
    to fp32 summation order.
Bar: the same plan gives the same bits; a different plan agrees within the output-rounding
bound (normwise 2e-3 for fp16), and both meet the 1e-2 bar against the CPU oracle on rows.
"""
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


def run_pair(M, K, Ns, seed, same_plan=True, rows=None):
    import torch

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


@pytest.mark.parametrize("first,second", [((16, 27648, [5120]), (8, 27648, [5120])),
                                          ((4, 27648, [5120]), (1, 27648, [5120])),
                                          ((100, 4096, [1024]), (90, 4096, [512]))])
def test_noalloc_equals_fused_twice(cuda, first, second):
    for i, (M, K, Ns) in enumerate((first, second)):
        run_pair(M, K, Ns, 7000 + 10 * i)


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
