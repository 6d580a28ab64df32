"""GPU test of concurrent calls on two streams: the library keeps one default workspace per
(device, stream), so calls whose plans meet through a workspace (X-resident and lockstep K
pieces, prefill stream-K) may run at the same time on different streams without sharing
arrival counters or partial tiles. Every result must equal the eager single-stream result of
the same plan, bit for bit.
"""
import pytest

import oracle as O
from gpu_util import DeviceProblem
from nebula_amd import hq

pytestmark = pytest.mark.gpu

SHAPES = [(O.INT4, O.F16, 4, 27648, 5120, "x 3 pieces"), (O.INT4, O.F16, 16, 27648, 5120, "hq_decode_ls_kernel<"),
          (O.INT4, O.F16, 100, 4096, 1024, "whole=0 stream-K")]


def test_two_streams_with_own_workspaces(cuda):
    import torch

    devs, refs = [], []
    for i, (fmt, xdt, M, K, N, plan) in enumerate(SHAPES):
        assert plan in hq.describe(fmt, xdt, M, K, N)
        D = DeviceProblem(O.Problem(fmt, M, K, N, 128, xdt, seed=9960 + i))
        devs.append(D)
        refs.append(D.run())
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outs = [[torch.empty_like(r) for r in refs] for _ in streams]
    for rep in range(6):
        for o in outs:
            for t in o:
                t.fill_(float("nan"))
        for s in streams:
            s.wait_stream(torch.cuda.current_stream())
        # The two streams issue the same three calls in opposite orders, interleaved.
        for j in range(len(SHAPES)):
            for k, s in enumerate(streams):
                i = j if k == 0 else len(SHAPES) - 1 - j
                D = devs[i]
                with torch.cuda.stream(s):
                    hq.gemm(D.P.fmt, D.X, D.Wp, D.S, D.P.N, 128, out=outs[k][i], stream=s)
        torch.cuda.synchronize()
        for k in range(len(streams)):
            for i, r in enumerate(refs):
                assert bool(torch.equal(outs[k][i], r)), f"stream {k}, shape {SHAPES[i][2:5]}, repetition {rep}"
