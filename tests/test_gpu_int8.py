"""GPU parity of the int8 path (hq_gemm_w8a8) against the oracle's restatement of
kernel_cutlass_int8_gemm (hydrogen/src/model/marlin_gemm.cu:327-377): activations quantised to
int8(clamp(x * 127)) toward zero, int8 weights q * 16 - 128 of int4 codes (:508), one scale per
column, y = scale * sum / 127.

The kernel sums the integer products exactly (int32); the reference accumulates fp32 quad by
quad. Both are checked against the exact value computed in float64 from the integer sums: the
kernel to one rounding of the output (two fp32 products), the oracle to its accumulation bound;
and the two against each other normwise (<= 1e-5).
"""
import os

import numpy as np
import pytest

import oracle as O
from nebula_amd import hq

pytestmark = pytest.mark.gpu


class w8_env:
    def __init__(self, **kv):
        self.kv = {f"HQ_W8_{k}": str(v) for k, v in kv.items()}

    def __enter__(self):
        self.old = {k: os.environ.get(k) for k in self.kv}
        os.environ.update(self.kv)

    def __exit__(self, *exc):
        for k, v in self.old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def problem(M, K, N, seed):
    rng = np.random.default_rng(seed)
    X = (rng.standard_normal((M, K)) * 0.5).astype(np.float32)  # N(0, 0.25), marlin_gemm.cu:473
    X[0, :7] = [np.nan, np.inf, -np.inf, 1.5, -1.5, 0.5, -0.5][: min(7, K)]  # clamps, NaN, truncation
    lin = O.gen_int4(seed, 1, K, N)
    W = O.int8_from_int4(lin, K, N)
    s = (0.05 + rng.integers(0, 1000, N) * 1e-4).astype(np.float32)  # marlin_gemm.cu:481-484
    return X, W, s


def quantize(X):
    # the oracle's quantiser on every distinct value (fast for the large shapes)
    vals, inv = np.unique(X.view(np.uint32), return_inverse=True)
    q = np.array([O.quantize_x_int8(v) for v in vals.view(np.float32)], dtype=np.int8)
    return q[inv].reshape(X.shape)


def exact(X, W, s):
    # integer sums in float64: exact (|sum| <= 128 * 128 * 27648 < 2^53)
    xq = quantize(X).astype(np.float64)
    wf = W.astype(np.float64)
    tot = xq @ wf
    absdot = np.abs(xq) @ np.abs(wf)
    return tot / 127.0 * s.astype(np.float64), absdot / 127.0 * np.abs(s.astype(np.float64))


def run(X, W, s, **kw):
    import torch

    M, K = X.shape
    N = W.shape[1]
    Wp = torch.from_numpy(hq.repack_int8(W)).cuda()
    y = hq.gemm_w8a8(torch.from_numpy(X).cuda(), Wp, torch.from_numpy(s).cuda(), N, **kw)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def check(y, X, W, s, what):
    K = X.shape[1]
    ex, mag = exact(X, W, s)
    # the kernel: exact int32 sum, then (float)sum * (1/127) * s: a few fp32 roundings
    assert np.all(np.abs(y - ex) <= 4 * 2.0**-24 * (np.abs(ex) + 1e-30) + 2.0**-24 * mag * 1e-7), what
    r = O.gemm_int8(X, W, s, threads=16)
    assert np.all(np.abs(r - ex) <= (K // 4 + 2) * 2.0**-24 * mag + 1e-30), what  # the oracle's own bound
    assert O.normwise_error(y, r) <= 1e-5, (what, O.normwise_error(y, r))


@pytest.mark.parametrize("M", [1, 3, 8, 16])
@pytest.mark.parametrize("K,N", [(128, 40), (1024, 1000), (5120, 5120), (4096, 4096), (27648, 512), (5120, 27648)])
def test_w8a8_default_plans(cuda, M, K, N):
    X, W, s = problem(M, K, N, M * 7 + K + N)
    y = run(X, W, s)
    if K * N > 5120 * 5120 and M not in (1, 8):
        # The call runs all M rows; the oracle checks the first, a middle and the last one (an
        # output row depends only on its own activation row; row 0 holds the special values).
        rows = sorted({0, M // 2, M - 1})
        check(y[rows], X[rows], W, s, f"M={M} K={K} N={N} rows {rows}")
    else:
        check(y, X, W, s, f"M={M} K={K} N={N}")


# Forced decompositions: slab widths, wavefront counts (some without k-blocks), K pieces
# (uneven, one k-block per piece); the int32 sums make every decomposition bit-identical.
@pytest.mark.parametrize("T,WK,S", [(2, 1, 1), (2, 8, 1), (4, 8, 1), (4, 3, 5), (2, 16, 16), (4, 8, 2), (2, 5, 3)])
@pytest.mark.parametrize("M", [1, 7, 16])
def test_w8a8_decompositions(cuda, T, WK, S, M):
    X, W, s = problem(M, 2048, 1000, 900 + M)
    y0 = run(X, W, s)
    with w8_env(T=T, WK=WK, S=S):
        y = run(X, W, s)
        y2 = run(X, W, s)
    assert np.array_equal(y.view(np.uint32), y0.view(np.uint32)), (T, WK, S, M)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    check(y, X, W, s, f"T={T} WK={WK} S={S} M={M}")


def test_w8a8_strided_rows_and_caller_workspace(cuda):
    import torch

    M, K, N = 5, 1024, 300
    X, W, s = problem(M, K, N, 77)
    Xs = torch.zeros((M, K + 36), dtype=torch.float32)
    Xs[:, :K] = torch.from_numpy(X)
    Xd = Xs.cuda()[:, :K]
    Wp = torch.from_numpy(hq.repack_int8(W)).cuda()
    Y = torch.full((M, N + 9), 7.0, device="cuda")
    with w8_env(S=4):  # K pieces: the counters must be left at zero for the next call
        need = hq.workspace_bytes_w8a8(M, K, N)
        ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
        hq.gemm_w8a8(Xd, Wp, torch.from_numpy(s).cuda(), N, out=Y[:, :N], workspace=ws)
        hq.gemm_w8a8(Xd, Wp, torch.from_numpy(s).cuda(), N, out=Y[:, :N], workspace=ws)
    torch.cuda.synchronize()
    assert int(ws[:4096].view(torch.int32).abs().sum().item()) == 0
    y = Y.cpu().numpy()
    assert np.all(y[:, N:] == 7.0)  # nothing written past N
    check(y[:, :N], X, W, s, "strided")


# One launch: when each thread has at most one 16-element unit of its K piece's rows, the GEMM
# quantises the fp32 rows itself; bit-identical to the quantisation launch (HQ_W8_QX = 0),
# including the NaN / infinity / clamp / truncation values of row 0.
@pytest.mark.parametrize("M,K,N,S", [(1, 5120, 1000, 0), (1, 128, 40, 0), (2, 2048, 700, 0), (3, 4096, 500, 3),
                                     (1, 27648, 512, 6)])
def test_w8a8_in_kernel_quantisation(cuda, M, K, N, S):
    X, W, s = problem(M, K, N, 1300 + M + K)
    env = {"S": S} if S else {}
    with w8_env(**env):
        y1 = run(X, W, s)
        with w8_env(QX=0):
            y0 = run(X, W, s)
    assert np.array_equal(y1.view(np.uint32), y0.view(np.uint32)), (M, K, N, S)
    check(y1, X, W, s, f"in-kernel quantisation M={M} K={K} S={S}")
