"""GPU parity of the general kernels: groups that are multiples of 32 but not of 128, and the
reference forward's per-group fp32 bias (hydrogen/include/marlin_gemm.hpp:100-107; the kernel
reads one scale and bias per 32-wide k chunk and forms w = q * s + b, hydrogen/src/model/
marlin_gemm.cu:191-196), against the oracle's restatement of the reference's host dequantisation
with that bias (marlin_gemm.cu:495-512) followed by the fp32 matmul (:60-69).

Bar: normwise 1e-2, the output-rounding bound (2e-3 fp16, 8e-3 bf16), and per element
|y - r| <= rel * |X| (|W| + |E|) + ulp(r), where E is the weight of code 8 of each group
(e = 8 s + b, which the kernels carry separately) and rel = 2^-10 (fp16) / 2^-7 (bf16).
A bias of exactly -8 s must give the same bits as no bias (the general kernels add e * sum x
with e = 0), and the general kernels agree with the fast ones (group 128, no bias) up to fp32
summation order.
"""
import os

import numpy as np
import pytest

import oracle as O
from gpu_util import to_dev_u16, to_dev_u32, to_host_f32
from nebula_amd import hq

pytestmark = pytest.mark.gpu

OUT_TOL = {O.F16: 2e-3, O.BF16: 8e-3}
REL = {O.F16: 2.0**-10, O.BF16: 2.0**-7}


class env:
    def __init__(self, **kv):
        self.kv = {k: str(v) for k, v in kv.items()}

    def __enter__(self):
        self.old = {k: os.environ.get(k) for k in self.kv}
        os.environ.update(self.kv)

    def __exit__(self, *exc):
        for k, v in self.old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


class Dev:
    def __init__(self, P):
        import torch

        self.P = P
        self.X = to_dev_u16(P.X, P.xdtype)
        self.S = to_dev_u16(P.scales)
        self.Wp = to_dev_u32(hq.repack(P.fmt, P.W, P.K, P.N))
        self.B = None if P.bias is None else torch.from_numpy(np.ascontiguousarray(P.bias)).cuda()

    def run(self, bias=True, X=None):
        return hq.gemm(self.P.fmt, self.X if X is None else X, self.Wp, self.S, self.P.N, self.P.group,
                       bias=self.B if bias else None)


def check(y, P, label, rows=None):
    yy = to_host_f32(y)
    ref = P.reference(rows=rows, threads=16)
    if rows is not None:
        yy = yy[rows]
    assert np.all(np.isfinite(yy)), label
    err = O.normwise_error(yy, ref)
    assert err <= OUT_TOL[P.xdtype], f"{label}: normwise {err:.3e}"
    X = O.to_f32(P.X if rows is None else P.X[rows], P.xdtype).astype(np.float64)
    if P.fmt == O.INT4:
        W = O.dequant_int4_bias(P.W, P.scales, P.bias, P.K, P.N, P.group).astype(np.float64)
        s = np.repeat(O.to_f32(P.scales, O.F16).astype(np.float64), P.group, axis=0)
        b = np.repeat(P.bias.astype(np.float64), P.group, axis=0) if P.bias is not None else -8.0 * s
        E = np.abs(8.0 * s + b)
    else:
        W = O.dequant(P.fmt, P.W, P.scales.ravel(), P.K, P.N, P.group).astype(np.float64)
        E = 0.0
    mag = np.abs(X) @ (np.abs(W) + E)
    ulp = np.abs(ref) * (2.0**-10 if P.xdtype == O.F16 else 2.0**-7) + 2.0**-24
    excess = np.abs(yy - ref) - (REL[P.xdtype] * mag + ulp)
    assert excess.max() <= 0, f"{label}: elementwise bound exceeded by {excess.max():.3e}"
    return err


FMTS = [(O.INT4, O.F16), (O.INT4, O.BF16), (O.TERNARY2, O.F16), (O.TERNARY2, O.BF16)]


@pytest.mark.parametrize("fmt,xdt", FMTS)
@pytest.mark.parametrize("g", [32, 64])
@pytest.mark.parametrize("M", [1, 4, 16, 40, 80])
def test_small_groups_decode(cuda, fmt, xdt, g, M):
    P = O.Problem(fmt, M, 2048, 1000, g, xdt, seed=6000 + M + g)
    check(Dev(P).run(), P, f"fmt={fmt} dt={xdt} g={g} M={M}")


@pytest.mark.parametrize("fmt,xdt", FMTS)
@pytest.mark.parametrize("g", [32, 64])
@pytest.mark.parametrize("M", [100, 300])
def test_small_groups_prefill(cuda, fmt, xdt, g, M):
    P = O.Problem(fmt, M, 1024, 520, g, xdt, seed=6100 + M + g)
    check(Dev(P).run(), P, f"prefill fmt={fmt} dt={xdt} g={g} M={M}")


@pytest.mark.parametrize("xdt", [O.F16, O.BF16])
@pytest.mark.parametrize("g", [32, 128, 256])
@pytest.mark.parametrize("M", [1, 8, 16, 33, 100, 257])
def test_random_bias(cuda, xdt, g, M):
    P = O.Problem(O.INT4, M, 1024, 700, g, xdt, seed=6200 + M + g, bias="random")
    check(Dev(P).run(), P, f"bias dt={xdt} g={g} M={M}")


@pytest.mark.parametrize("xdt", [O.F16, O.BF16])
@pytest.mark.parametrize("g", [64, 128])
@pytest.mark.parametrize("M", [1, 16, 80, 200])
def test_bias_minus_8s_same_bits_as_no_bias(cuda, xdt, g, M):
    import torch

    P = O.Problem(O.INT4, M, 1024, 520, g, xdt, seed=6300 + M + g, bias="minus8s")
    D = Dev(P)
    with env(HQ_GENERAL=1):  # the general kernels also without a bias (group 128)
        yb = D.run(bias=True)
        y0 = D.run(bias=False)
    assert bool(torch.equal(yb, y0)), f"dt={xdt} g={g} M={M}"
    check(yb, P, f"bias -8s dt={xdt} g={g} M={M}")


@pytest.mark.parametrize("fmt,xdt", FMTS)
@pytest.mark.parametrize("M", [1, 16, 64, 300])
def test_general_kernels_agree_with_fast_kernels(cuda, fmt, xdt, M):
    P = O.Problem(fmt, M, 2048, 640, 128, xdt, seed=6400 + M)
    D = Dev(P)
    y_fast = D.run()
    with env(HQ_GENERAL=1):
        assert "general" in hq.describe(fmt, xdt, M, 2048, 640)
        y_gen = D.run()
    a, b = to_host_f32(y_gen), to_host_f32(y_fast)
    assert O.normwise_error(a, b) <= OUT_TOL[xdt]
    check(y_gen, P, f"general fmt={fmt} dt={xdt} M={M}")


@pytest.mark.parametrize("M", [4, 16, 80])
def test_bias_with_split_slabs(cuda, M):
    # 27648 x 5120: 40 eight-tile slabs, each cut along K into pieces summed by the fix-up.
    P = O.Problem(O.INT4, M, 27648, 5120, 128, O.F16, seed=6500 + M, bias="random")
    assert "pieces" in hq.describe(O.INT4, O.F16, M, 27648, 5120, with_bias=True)
    check(Dev(P).run(), P, f"split slabs bias M={M}")


@pytest.mark.parametrize("psk", [0, 24])
def test_small_group_prefill_stream_k(cuda, psk):
    P = O.Problem(O.INT4, 100, 4096, 1024, 64, O.BF16, seed=6600, bias="random")
    D = Dev(P)
    with env(HQ_PREFILL_PSK=psk) if psk else env():
        y = D.run()
    check(y, P, f"prefill stream-K g=64 psk={psk}")


@pytest.mark.parametrize("M", [1, 16, 80, 300])
def test_fused_mixed_bias_segments(cuda, M):
    # One segment with a bias, one without (zero point 8), groups of 64: one fused call.
    Ns = [600, 1000]
    probs = [O.Problem(O.INT4, M, 1024, Ns[0], 64, O.F16, seed=6700 + M, bias="random"),
             O.Problem(O.INT4, M, 1024, Ns[1], 64, O.F16, seed=6710 + M)]
    probs[1].X = probs[0].X
    devs = [Dev(p) for p in probs]
    segs = [(devs[0].Wp, devs[0].S, Ns[0], devs[0].B), (devs[1].Wp, devs[1].S, Ns[1])]
    outs = hq.gemm_fused(O.INT4, devs[0].X, segs, group=64)
    for p, y in zip(probs, outs):
        check(y, p, f"fused mixed bias M={M} N={p.N}")


def test_decode_27b_shape_bias(cuda):
    P = O.Problem(O.INT4, 16, 5120, 27648, 128, O.F16, seed=6800, bias="random")
    y = Dev(P).run()
    rows = np.arange(16)
    check(y, P, "K=5120 N=27648 M=16 bias", rows=rows)
