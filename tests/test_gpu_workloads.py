"""GPU parity at the benchmark workloads themselves, with the plans the library picks for them.

Every case runs the default plan of its exact shape (no forced decomposition) and compares
with the CPU oracle (restated dequantize-then-matmul of hydrogen/src/model/marlin_gemm.cu:
495-512 and 60-69). Bar: normwise max relative error <= 1e-2 (the target operator's), and
the tighter output-rounding bound OUT_TOL; where the oracle cost allows, the per-element bound
|y - r| <= 2^-10 (|X| |W|) + ulp(r) as well (2^-7 for bf16).

Workloads:
  * decode sweep, int4 fp16, (K, N) in {(5120, 27648), (27648, 5120)}, M in {1, 2, 4, 8, 16}
    (the X-resident kernel in pairs of whole 4-tile slabs on 5120 x 27648 at every M, with
    whole slabs at M <= 2 and K cut in three pieces at M = 4 and 8 on 27648 x 5120, the
    lockstep kernel at M = 16 on 27648 x 5120);
  * prefill, int4 fp16, K = 5120, N = 27648, M = 4096, every row;
  * the split-fuse mixed batch, M = 1024 = 1008 prefill-chunk rows + 16 decode rows, in both
    orders (hydrogen/src/batcher/split_fuse.cpp:110-159 puts the decode rows first):
      (a) fused QKV, int4, K = 5120, N = 5120 | 1024 | 1024;
      (b) fused gate||up, ternary, K = 5120, N = 27648 | 27648;
    both group 128, fp16 activations.
"""
import numpy as np
import pytest

import oracle as O
from gpu_util import DeviceProblem, to_dev_u16, to_host_f32
from nebula_amd import hq

pytestmark = pytest.mark.gpu

OUT_TOL = {O.F16: 2e-3, O.BF16: 8e-3}
BAR = 1e-2
ELEM_REL = {O.F16: 2.0**-10, O.BF16: 2.0**-7}


def elementwise_ok(y, ref, P, rows=None):
    """Per-element bound |y - r| <= rel (|X| |W|) + ulp_out(r) over the given rows (float64)."""
    X = O.to_f32(P.X if rows is None else P.X[rows], P.xdtype).astype(np.float64)
    W = O.dequant(P.fmt, P.W, P.scales.ravel(), P.K, P.N, P.group)
    mag = np.abs(X) @ np.abs(W).astype(np.float64)
    out_ulp = np.abs(ref) * (2.0**-10 if P.xdtype == O.F16 else 2.0**-7) + 2.0**-24
    excess = np.abs(y.astype(np.float64) - ref) - (ELEM_REL[P.xdtype] * mag + out_ulp)
    return float(excess.max())


def compare(y, ref, P, label, rows=None, elementwise=True):
    yy = to_host_f32(y) if not isinstance(y, np.ndarray) else y
    if rows is not None:
        yy = yy[rows]
    assert np.all(np.isfinite(yy)), f"{label}: non-finite outputs"
    err = O.normwise_error(yy, ref)
    assert err <= BAR, f"{label}: normwise {err:.3e} > {BAR}"
    assert err <= OUT_TOL[P.xdtype], f"{label}: normwise {err:.3e} > {OUT_TOL[P.xdtype]}"
    if elementwise:
        ex = elementwise_ok(yy, ref, P, rows)
        assert ex <= 0, f"{label}: elementwise bound exceeded by {ex:.3e}"
    return err


@pytest.mark.parametrize("K,N", [(5120, 27648), (27648, 5120)])
@pytest.mark.parametrize("M", [1, 2, 4, 8, 16])
def test_decode_sweep_large_shapes(cuda, K, N, M):
    P = O.Problem(O.INT4, M, K, N, 128, O.F16, seed=5000 + M + K // 1000)
    D = DeviceProblem(P)
    y = D.run()
    compare(y, P.reference(threads=16), P, f"decode K={K} N={N} M={M}")
    # Bit-reproducible from call to call (fixed summation order, also through the fix-up).
    assert bool((D.run() == y).all())


def test_decode_sweep_5120_square_m1_m16(cuda):
    for M in (1, 16):
        P = O.Problem(O.INT4, M, 5120, 5120, 128, O.F16, seed=5100 + M)
        compare(DeviceProblem(P).run(), P.reference(threads=16), P, f"decode 5120x5120 M={M}")


def test_prefill_m4096(cuda):
    M, K, N = 4096, 5120, 27648
    P = O.Problem(O.INT4, M, K, N, 128, O.F16, seed=5200)
    y = to_host_f32(DeviceProblem(P).run())
    rows = np.arange(M)
    compare(y, P.reference(rows=rows, threads=16), P, "prefill M=4096", rows=rows)


def mixed_rows(order, seed, K):
    """1008 prefill-chunk rows and 16 decode rows (independent draws), concatenated in the
    given order; returns the fp16 bits [1024, K] and where the decode rows went."""
    pre = O.gen_normal(seed, 21, 1008 * K, 1.0, False, O.F16).reshape(1008, K)
    dec = O.gen_normal(seed, 22, 16 * K, 1.0, False, O.F16).reshape(16, K)
    if order == "decode_first":
        return np.concatenate([dec, pre]), np.arange(16)
    return np.concatenate([pre, dec]), np.arange(1008, 1024)


def run_mixed(fmt, Ns, order, seed):
    K, M = 5120, 1024
    Xb, dec_rows = mixed_rows(order, seed, K)
    probs = []
    for i, n in enumerate(Ns):
        p = O.Problem(fmt, 1, K, n, 128, O.F16, seed=seed + i)
        p.X, p.M = Xb, M
        probs.append(p)
    devs = [DeviceProblem(p) for p in probs]
    outs = hq.gemm_fused(fmt, to_dev_u16(Xb, O.F16), [(d.Wp, d.S, d.P.N) for d in devs])
    return probs, [to_host_f32(y) for y in outs], dec_rows


@pytest.mark.parametrize("order", ["decode_first", "prefill_first"])
def test_mixed_batch_fused_qkv_int4(cuda, order):
    Ns = [5120, 1024, 1024]
    probs, outs, dec_rows = run_mixed(O.INT4, Ns, order, 5300)
    rng = np.random.default_rng(5301)
    rows = np.sort(np.concatenate([dec_rows[rng.choice(16, 4, replace=False)],
                                   rng.choice(np.setdiff1d(np.arange(1024), dec_rows), 28, replace=False)]))
    for P, y in zip(probs, outs):
        compare(y, P.reference(rows=rows, threads=16), P, f"QKV {order} N={P.N}", rows=rows)


@pytest.mark.parametrize("order", ["decode_first", "prefill_first"])
def test_mixed_batch_fused_gate_up_ternary(cuda, order):
    Ns = [27648, 27648]
    probs, outs, dec_rows = run_mixed(O.TERNARY2, Ns, order, 5400)
    rng = np.random.default_rng(5401)
    rows = np.sort(np.concatenate([dec_rows[rng.choice(16, 3, replace=False)],
                                   rng.choice(np.setdiff1d(np.arange(1024), dec_rows), 13, replace=False)]))
    for P, y in zip(probs, outs):
        compare(y, P.reference(rows=rows, threads=16), P, f"gate||up {order} N={P.N}", rows=rows)


def test_mixed_batch_row_order_does_not_matter(cuda):
    # The same 1024 rows in the two orders give the same outputs per row (each output is one
    # fp32 chain over K; a different tile position may change the K split, so up to fp32
    # summation order).
    Ns = [5120, 1024, 1024]
    _, a, _ = run_mixed(O.INT4, Ns, "decode_first", 5500)
    _, b, _ = run_mixed(O.INT4, Ns, "prefill_first", 5500)
    perm = np.concatenate([np.arange(1008, 1024), np.arange(1008)])  # prefill-first row of each decode-first row
    for ya, yb in zip(a, b):
        yb = yb[perm]
        assert float(np.abs(ya - yb).max() / np.abs(yb).max()) <= 2 * 2.0**-11
