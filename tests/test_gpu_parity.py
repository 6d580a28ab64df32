"""GPU parity of the HIP qGEMM against the CPU oracle, called through the C ABI.

Bar of the target operator: max relative error <= 1e-2 with fp32 accumulation on both sides,
measured normwise (max |y - r| / max |r|); the integer/byte work (repacks) is bit-exact.
Two tighter checks stop a bug from hiding under that bar:
  * normwise error <= OUT_TOL[dtype] (output rounding: fp16 2^-11, bf16 2^-8, plus slack);
  * per element, |y - r| <= 2^-10 * (|X| |W|)[m, n] + ulp(r): the prefill kernel rounds
    each scaled weight (q - 8) * s to fp16/bf16 once (relative 2^-11 / 2^-8) before the
    MFMA, the decode kernel applies the scale in fp32, and both accumulate in fp32.
    bf16 uses 2^-7 in place of 2^-10.
"""
import numpy as np
import pytest

import oracle as O
from gpu_util import DeviceProblem, assert_parity, to_dev_u16, to_dev_u32, to_host_f32
from nebula_amd import hq

pytestmark = pytest.mark.gpu

OUT_TOL = {O.F16: 2e-3, O.BF16: 8e-3}
BAR = 1e-2


ELEM_REL = {O.F16: 2.0**-10, O.BF16: 2.0**-7}


def elementwise_bound_check(y, ref, P, rows=None):
    """|y - r| <= rel * (|X| |W|) + ulp_out(r), evaluated in float64 (small and medium shapes)."""
    X = O.to_f32(P.X if rows is None else P.X[rows], P.xdtype).astype(np.float64)
    W = O.dequant(P.fmt, P.W, P.scales.ravel(), P.K, P.N, P.group).astype(np.float64)
    mag = np.abs(X) @ np.abs(W)
    yy = to_host_f32(y) if not isinstance(y, np.ndarray) else y
    out_ulp = np.abs(ref) * (2.0**-10 if P.xdtype == O.F16 else 2.0**-7) + 2.0**-24
    excess = np.abs(yy - ref) - (ELEM_REL[P.xdtype] * mag + out_ulp)
    assert np.all(excess <= 0), f"elementwise bound exceeded by {excess.max():.3e} at {np.unravel_index(excess.argmax(), excess.shape)}"


def check(y, ref, xdtype, label, P=None):
    err = assert_parity(y, ref, BAR, label)
    assert err <= OUT_TOL[xdtype], f"{label}: normwise {err:.3e} above output-rounding bound {OUT_TOL[xdtype]}"
    if P is not None and P.M * P.K * P.N <= 4e9:
        elementwise_bound_check(y, ref, P)
    return err


def test_w4a16_m16_4096(cuda):
    # The single W4A16 GEMM: M=16, K=N=4096, int4 zero point 8, g=128, fp16 in/out.
    P = O.Problem(O.INT4, 16, 4096, 4096, 128, O.F16, seed=42)
    D = DeviceProblem(P)
    check(D.run(), P.reference(), O.F16, "c0", P)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 11, 16])
def test_decode_m_sweep_int4_f16(cuda, M):
    P = O.Problem(O.INT4, M, 5120, 5120, 128, O.F16, seed=100 + M)
    check(DeviceProblem(P).run(), P.reference(), O.F16, f"int4 f16 M={M}", P)


@pytest.mark.parametrize("M", [1, 4, 16])
def test_decode_int4_bf16(cuda, M):
    P = O.Problem(O.INT4, M, 2048, 1536, 128, O.BF16, seed=200 + M)
    check(DeviceProblem(P).run(), P.reference(), O.BF16, f"int4 bf16 M={M}", P)


@pytest.mark.parametrize("M", [1, 8])
def test_ternary_bf16_decode_27b(cuda, M):
    # Ternary decode GEMV: ternary {-1,0,1} p={.25,.5,.25}, K=5120, N=27648, bf16 activations.
    P = O.Problem(O.TERNARY2, M, 5120, 27648, 128, O.BF16, seed=300 + M)
    check(DeviceProblem(P).run(), P.reference(), O.BF16, f"ternary bf16 M={M}", P)


@pytest.mark.parametrize("M", [1, 16])
def test_decode_ternary_f16(cuda, M):
    P = O.Problem(O.TERNARY2, M, 1024, 2048, 128, O.F16, seed=310 + M)
    check(DeviceProblem(P).run(), P.reference(), O.F16, f"ternary f16 M={M}", P)


@pytest.mark.parametrize("K,N", [(5120, 27648), (27648, 5120)])
def test_w4a16_27b_shapes_m16(cuda, K, N):
    P = O.Problem(O.INT4, 16, K, N, 128, O.F16, seed=400)
    check(DeviceProblem(P).run(), P.reference(threads=16), O.F16, f"w4a16 {K}x{N} M=16")


@pytest.mark.parametrize("fmt,xdt", [(O.INT4, O.F16), (O.INT4, O.BF16), (O.TERNARY2, O.F16), (O.TERNARY2, O.BF16)])
@pytest.mark.parametrize("N", [1, 20, 1000])
def test_ragged_n(cuda, fmt, xdt, N):
    P = O.Problem(fmt, 3, 384, N, 128, xdt, seed=500 + N)
    check(DeviceProblem(P).run(), P.reference(), xdt, f"ragged N={N}", P)


@pytest.mark.parametrize("group", [256, 512])
def test_larger_groups(cuda, group):
    P = O.Problem(O.INT4, 7, 2048, 640, group, O.F16, seed=600 + group)
    check(DeviceProblem(P).run(), P.reference(), O.F16, f"group {group}", P)


def test_golden_fixture(cuda):
    from pathlib import Path

    data = np.load(Path(__file__).resolve().parent / "golden" / "qgemm_small.npz")
    for case in sorted({k.split("/")[0] for k in data.files}):
        fmt, xdt = int(data[f"{case}/fmt"]), int(data[f"{case}/xdtype"])
        X, W, S, N, g = data[f"{case}/X"], data[f"{case}/W"], data[f"{case}/scales"], int(data[f"{case}/N"]), int(
            data[f"{case}/group"])
        K = X.shape[1]
        Wp = to_dev_u32(hq.repack(fmt, W, K, N))
        y = hq.gemm(fmt, to_dev_u16(X, xdt), Wp, to_dev_u16(S), N, g)
        check(y, data[f"{case}/Y64"], xdt, case)


@pytest.mark.parametrize("kernel", [0, 1])
def test_zero_point_and_one_hot_exact(cuda, kernel):
    with decode_env(KERNEL=kernel):
        zero_point_and_one_hot(cuda)


def zero_point_and_one_hot(cuda):
    K, N = 512, 48
    P = O.Problem(O.INT4, 1, K, N, 128, O.F16, seed=700)
    ks = [0, 7, 8, 127, 128, 300, 511]
    X = np.zeros((len(ks), K), dtype=np.uint16)
    for r, k in enumerate(ks):
        X[r, k] = 0x3C00
    D = DeviceProblem(P)
    y = to_host_f32(D.run(X=to_dev_u16(X, O.F16)))
    Wdq = O.dequant(O.INT4, P.W, P.scales.ravel(), K, N, 128)
    expect = O.to_f32(O.from_f32(Wdq[ks], O.F16), O.F16)  # the dequantised row, rounded to fp16 once
    assert np.array_equal(y, expect)
    # All weights at the zero point. The decode kernels dequantise int4 to magic + q (magic
    # 1024 or 64 per fragment word) and remove magic + 8 with correction MFMAs, so q = 8
    # leaves only the fp32 rounding of per-k-block sums of at most 1032 |x| (8 MFMAs, each
    # rounding at most twice): |y| <= 16 * 2^-24 * 1032 * sum_kb (sum|x|) s.
    W8 = np.full((K // 8) * N, 0x88888888, dtype=np.uint32)
    y0 = to_host_f32(hq.gemm(O.INT4, D.X, to_dev_u32(hq.repack(O.INT4, W8, K, N)), D.S, N))
    xsum = np.abs(O.to_f32(P.X, O.F16).astype(np.float64)).reshape(P.M, K // 128, 128).sum(-1)
    s = O.to_f32(P.scales, O.F16).astype(np.float64).reshape(K // 128, N)
    bound = 16 * 2.0**-24 * 1032 * xsum @ np.abs(s)
    assert np.all(np.abs(y0) <= bound), np.abs(y0).max()
    assert np.abs(y0).max() < 1e-3


@pytest.mark.parametrize("M,xdt", [(4, O.BF16), (4, O.F16), (40, O.F16), (100, O.BF16), (300, O.F16), (300, O.BF16)])
def test_ternary_nonfinite_scale_drops_group(cuda, M, xdt):
    # Decode (M <= 16) and every prefill tile shape (64, 128, 256 rows, stream-K at M = 300).
    P = O.Problem(O.TERNARY2, M, 512, 64, 128, xdt, seed=710 + M)
    P.scales[1, 5] = 0x7E00
    P.scales[2, 9] = 0x7C00
    P.scales[3, 60] = 0xFC00
    check(DeviceProblem(P).run(), P.reference(), xdt, f"nonfinite scale M={M}")


def test_strided_operands(cuda):
    import torch

    P = O.Problem(O.INT4, 5, 1024, 200, 128, O.F16, seed=720)
    D = DeviceProblem(P)
    Xw = torch.zeros((5, 1024 + 64), dtype=torch.float16, device="cuda")
    Xw[:, :1024] = D.X
    Yw = torch.full((5, 256), 7.0, dtype=torch.float16, device="cuda")
    hq.gemm(O.INT4, Xw[:, :1024], D.Wp, D.S, 200, out=Yw[:, :200])
    check(Yw[:, :200], P.reference(), O.F16, "strided")
    assert torch.all(Yw[:, 200:] == 7.0)


@pytest.mark.parametrize("M", [17, 40, 64, 65, 100, 128, 129, 256, 300])
def test_prefill_m_sweep(cuda, M):
    P = O.Problem(O.INT4, M, 1024, 520, 128, O.F16, seed=800 + M)
    check(DeviceProblem(P).run(), P.reference(), O.F16, f"M={M}", P)


@pytest.mark.parametrize("fmt,xdt", [(O.INT4, O.BF16), (O.TERNARY2, O.F16), (O.TERNARY2, O.BF16)])
@pytest.mark.parametrize("M", [33, 257])
def test_prefill_formats(cuda, fmt, xdt, M):
    P = O.Problem(fmt, M, 768, 300, 128, xdt, seed=850 + M)
    check(DeviceProblem(P).run(), P.reference(), xdt, f"prefill fmt={fmt} dt={xdt} M={M}", P)


def test_prefill_group_256(cuda):
    P = O.Problem(O.INT4, 200, 1024, 256, 256, O.F16, seed=870)
    check(DeviceProblem(P).run(), P.reference(), O.F16, "prefill g256", P)


@pytest.mark.parametrize("fmt,xdt,M,K,N", [(O.INT4, O.F16, 160, 4096, 40960), (O.INT4, O.BF16, 136, 5120, 34816)])
def test_prefill_64_row_tiles_default_plan(cuda, fmt, xdt, M, K, N):
    # 128-row tiles a few past one per CU: the default plan runs 64-row tiles, two per CU
    # (asserted on 256-CU devices); rows at every band boundary against the oracle.
    import torch

    desc = hq.describe(fmt, xdt, M, K, N)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert "64-row tiles=" in desc and "stream-K workgroups=0" in desc, desc
    P = O.Problem(fmt, M, K, N, 128, xdt, seed=4200 + M)
    y = to_host_f32(DeviceProblem(P).run())
    rows = np.array(sorted({0, 1, 63, 64, 65, 127, 128, M - 2, M - 1}))
    ref = P.reference(rows=rows, threads=16)
    assert O.normwise_error(y[rows], ref) <= OUT_TOL[xdt], desc
    elementwise_bound_check(y[rows], ref, P, rows=rows)


@pytest.mark.parametrize("M,nrows", [(512, 0), (2048, 0)])
def test_prefill_27b(cuda, M, nrows):
    # The prefill shape (K=5120, N=27648) at M = 512 and 2048, every row against the oracle,
    # normwise and element by element.
    P = O.Problem(O.INT4, M, 5120, 27648, 128, O.F16, seed=880 + M)
    y = to_host_f32(DeviceProblem(P).run())
    rows = np.arange(M) if nrows == 0 else np.sort(np.random.default_rng(M).choice(M, size=nrows, replace=False))
    ref = P.reference(rows=rows, threads=16)
    err = O.normwise_error(y[rows], ref)
    assert err <= OUT_TOL[O.F16], f"prefill K=5120 N=27648 M={M}: {err:.3e}"
    elementwise_bound_check(y[rows], ref, P, rows=rows)


def test_rows_independent_and_deterministic(cuda):
    P = O.Problem(O.INT4, 16, 2048, 1024, 128, O.F16, seed=900)
    D = DeviceProblem(P)
    y16 = D.run()
    y16b = D.run()
    assert torch_equal(y16, y16b)
    for r in (0, 7, 15):
        y1 = D.run(X=D.X[r:r + 1].contiguous())
        np.testing.assert_allclose(to_host_f32(y1)[0], to_host_f32(y16)[r], rtol=2e-3, atol=1e-3)


def torch_equal(a, b):
    import torch

    return bool(torch.equal(a, b))


@pytest.mark.parametrize("fmt,xdt,Ns", [(O.INT4, O.F16, [5120, 1024, 1024]), (O.TERNARY2, O.F16, [2048, 2048]),
                                        (O.INT4, O.BF16, [640, 33])])
@pytest.mark.parametrize("M", [1, 16, 80])
def test_fused_equals_separate(cuda, fmt, xdt, Ns, M):
    K = 1024
    probs = [O.Problem(fmt, M, K, n, 128, xdt, seed=1000 + i) for i, n in enumerate(Ns)]
    for p in probs[1:]:
        p.X = probs[0].X
    devs = [DeviceProblem(p) for p in probs]
    X = devs[0].X
    outs = hq.gemm_fused(fmt, X, [(d.Wp, d.S, d.P.N) for d in devs])
    for d, y in zip(devs, outs):
        # Same values up to fp32 summation order (the fused launch may split K differently).
        sep = to_host_f32(d.run(X=X))
        assert O.normwise_error(to_host_f32(y), sep) <= OUT_TOL[xdt]
        check(y, d.P.reference(), xdt, f"fused N={d.P.N}", d.P)


@pytest.mark.parametrize("fmt", [O.INT4, O.TERNARY2])
def test_device_repack_matches_host(cuda, fmt):
    import torch

    K, N = 1024, 300
    W = O.gen_int4(5, 5, K, N) if fmt == O.INT4 else O.gen_ternary(5, 5, K, N)
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    dev = hq.repack_device(fmt, to_dev_u32(W), K, N, bad_flag=flag)
    torch.cuda.synchronize()
    host = hq.repack(fmt, W, K, N)
    assert np.array_equal(dev.cpu().numpy().view(np.uint32), host)
    assert int(flag.item()) == 0
    if fmt == O.TERNARY2:
        W[7] |= 3 << 4
        hq.repack_device(fmt, to_dev_u32(W), K, N, bad_flag=flag)
        torch.cuda.synchronize()
        assert int(flag.item()) == 1


# ---------------------------------------------------------------- decode work decomposition
# Keys of the per-wavefront kernel's decomposition; forcing any of them also selects that
# kernel (HQ_DECODE_KERNEL=0), which otherwise serves only M <= 4.
_PW_KEYS = {"T", "WK", "P", "G", "U", "CONTIG"}


class decode_env:
    """Force the decode kernel (KERNEL=0 per-wavefront, 1 lockstep) and its decomposition
    for a block: per-wavefront slab width T, wavefronts WK, workgroups P, ring depth U;
    lockstep LS_KG (k-groups), LS_T (tiles per wavefront), LS_U (steps in flight), LS_S
    (pieces per slab)."""

    def __init__(self, **kv):
        if "KERNEL" not in kv and _PW_KEYS & set(kv):
            kv["KERNEL"] = 0
        self.kv = {f"HQ_DECODE_{k}": str(v) for k, v in kv.items()}

    def __enter__(self):
        import os

        self.old = {k: os.environ.get(k) for k in self.kv}
        os.environ.update(self.kv)

    def __exit__(self, *exc):
        import os

        for k, v in self.old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


# (T, WK, P): one workgroup for everything, grids that cut every slab several times (with
# wavefronts left without units in short pieces), and grids aligned to the slabs.
DECOMP = [(4, 8, 1), (4, 8, 7), (4, 3, 64), (4, 8, 256), (4, 1, 997), (2, 8, 30), (2, 5, 513), (1, 16, 63),
          (1, 3, 300), (4, 8, 16), (8, 8, 8), (8, 4, 3), (8, 2, 100)]


@pytest.mark.parametrize("contig", [0, 1])
@pytest.mark.parametrize("T,WK,Pg", DECOMP)
@pytest.mark.parametrize("M", [1, 7, 16])
def test_decode_decompositions_int4(cuda, T, WK, Pg, M, contig):
    # K = 2048 (16 k-blocks), N = 1000 (63 tiles, ragged): 16 slabs of 4 tiles. contig
    # selects contiguous per-wavefront k runs instead of interleaved k-blocks.
    P = O.Problem(O.INT4, M, 2048, 1000, 128, O.F16, seed=2000 + M)
    D = DeviceProblem(P)
    with decode_env(T=T, WK=WK, P=Pg, CONTIG=contig):
        y = D.run()
    check(y, P.reference(), O.F16, f"T={T} WK={WK} P={Pg} M={M} contig={contig}", P)


# Register ring depths (k-blocks in flight per wavefront) other than each slab width's
# default: the same per-wavefront k order, so the same bits as the default depth.
@pytest.mark.parametrize("fmt,xdt", [(O.INT4, O.F16), (O.TERNARY2, O.BF16)])
@pytest.mark.parametrize("T,U", [(8, 3), (4, 2), (4, 4), (2, 2), (2, 4)])
def test_decode_ring_depths(cuda, fmt, xdt, T, U):
    P = O.Problem(fmt, 5, 2048, 1000, 128, xdt, seed=2150 + T * 10 + U)
    D = DeviceProblem(P)
    with decode_env(T=T, WK=4, P=23):
        y_default = D.run()
        with decode_env(U=U):
            y = D.run()
    assert torch_equal(y, y_default)
    check(y, P.reference(), xdt, f"fmt={fmt} T={T} U={U}", P)


@pytest.mark.parametrize("fmt,xdt", [(O.INT4, O.BF16), (O.TERNARY2, O.F16), (O.TERNARY2, O.BF16)])
@pytest.mark.parametrize("T,WK,Pg,contig", [(4, 8, 5, 0), (2, 4, 77, 1), (1, 16, 200, 0), (4, 3, 40, 1), (8, 8, 6, 1),
                                             (8, 3, 50, 0)])
def test_decode_decompositions_formats(cuda, fmt, xdt, T, WK, Pg, contig):
    P = O.Problem(fmt, 9, 1536, 700, 256, xdt, seed=2100)
    D = DeviceProblem(P)
    with decode_env(T=T, WK=WK, P=Pg, CONTIG=contig):
        y = D.run()
    check(y, P.reference(), xdt, f"fmt={fmt} T={T} WK={WK} P={Pg}", P)


@pytest.mark.parametrize("Pg", [3, 50, 333])
def test_decode_fused_decompositions(cuda, Pg):
    # Ranges that start in one segment and end in the next.
    Ns, K, M = [600, 130, 1000], 1024, 5
    probs = [O.Problem(O.INT4, M, K, n, 128, O.F16, seed=2200 + i) for i, n in enumerate(Ns)]
    for p in probs[1:]:
        p.X = probs[0].X
    devs = [DeviceProblem(p) for p in probs]
    with decode_env(P=Pg):
        outs = hq.gemm_fused(O.INT4, devs[0].X, [(d.Wp, d.S, d.P.N) for d in devs])
    for d, y in zip(devs, outs):
        check(y, d.P.reference(), O.F16, f"fused P={Pg} N={d.P.N}", d.P)


def test_decode_caller_workspace_reused(cuda):
    import torch

    K, N = 27648, 5120
    P16 = O.Problem(O.INT4, 16, K, N, 128, O.F16, seed=2300)
    D = DeviceProblem(P16)
    need = hq.workspace_bytes(O.INT4, 16, K, N)
    assert need > 0
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    y_int = D.run()
    y_ws = hq.gemm(O.INT4, D.X, D.Wp, D.S, N, workspace=ws)
    assert torch_equal(y_ws, y_int)  # same decomposition, fixed summation order
    # Second call on the same workspace with fewer rows: counters were left at zero.
    y_ws4 = hq.gemm(O.INT4, D.X[:4].contiguous(), D.Wp, D.S, N, workspace=ws)
    assert torch_equal(y_ws4, D.run(X=D.X[:4].contiguous()))
    check(y_ws, P16.reference(), O.F16, "caller workspace")
    torch.cuda.synchronize()
    assert int(ws[:4 * ((N + 15) // 16)].view(torch.int32).abs().sum().item()) == 0


# Variable-width slabs: G slabs split each segment's tiles as evenly as integers allow
# (63 tiles here), with whole slabs per workgroup (P = G) or cut slabs (P != G).
@pytest.mark.parametrize("T,G,WK,Pg", [(8, 10, 4, 10), (8, 9, 3, 7), (8, 10, 4, 23), (4, 20, 2, 20), (4, 17, 4, 40),
                                       (2, 40, 4, 40), (2, 35, 1, 12)])
@pytest.mark.parametrize("M", [1, 16])
def test_decode_variable_slabs(cuda, T, G, WK, Pg, M):
    P = O.Problem(O.INT4, M, 2048, 1000, 128, O.F16, seed=2400 + M)
    D = DeviceProblem(P)
    with decode_env(T=T, G=G, WK=WK, P=Pg):
        y = D.run()
    check(y, P.reference(), O.F16, f"T={T} G={G} WK={WK} P={Pg} M={M}", P)


@pytest.mark.parametrize("G,Pg", [(12, 12), (12, 29)])
def test_decode_variable_slabs_fused(cuda, G, Pg):
    Ns, K, M = [600, 130, 1000], 1024, 3
    probs = [O.Problem(O.TERNARY2, M, K, n, 128, O.BF16, seed=2500 + i) for i, n in enumerate(Ns)]
    for p in probs[1:]:
        p.X = probs[0].X
    devs = [DeviceProblem(p) for p in probs]
    with decode_env(T=8, G=G, P=Pg):
        outs = hq.gemm_fused(O.TERNARY2, devs[0].X, [(d.Wp, d.S, d.P.N) for d in devs])
    for d, y in zip(devs, outs):
        check(y, d.P.reference(), O.BF16, f"fused variable slabs G={G} P={Pg} N={d.P.N}", d.P)


# ---------------------------------------------------------------- lockstep decode kernel
# (KG, T, U, S): every instantiated (k-groups, tiles per wavefront, steps in flight), with
# whole slabs (S = 1) and K splits into 2..8 pieces (S = 3 and 5 cut 16 k-blocks unevenly;
# with four k-groups and 3-4 k-blocks per piece some k-groups get none).
LS_CFGS = [(1, 2, 4, 1), (2, 1, 4, 1), (2, 2, 2, 1), (2, 2, 3, 1), (2, 4, 2, 1), (4, 1, 3, 1), (4, 2, 2, 1),
           (4, 2, 3, 1), (2, 2, 2, 3), (2, 2, 3, 8), (4, 2, 2, 5), (2, 1, 4, 2), (1, 2, 4, 4)]


@pytest.mark.parametrize("KG,T,U,S", LS_CFGS)
@pytest.mark.parametrize("M", [4, 7, 16])
def test_lockstep_configs_int4(cuda, KG, T, U, S, M):
    # K = 2048 (16 k-blocks), N = 1000 (63 tiles: the last slab is partial for every width).
    P = O.Problem(O.INT4, M, 2048, 1000, 128, O.F16, seed=3000 + M)
    D = DeviceProblem(P)
    with decode_env(KERNEL=1, LS_KG=KG, LS_T=T, LS_U=U, LS_S=S):
        y = D.run()
        y2 = D.run()
    assert torch_equal(y, y2)  # fixed summation order: bit-identical from run to run
    check(y, P.reference(), O.F16, f"KG={KG} T={T} U={U} S={S} M={M}", P)


# Slabs narrower than GW * T tiles (SW): the last wavefronts own fewer tiles or none, and the
# tiles past a slab belong to the next one (they must read zero and never be stored).
@pytest.mark.parametrize("KG,T,U,S,SW", [(2, 2, 2, 1, 7), (2, 2, 2, 1, 5), (2, 2, 3, 3, 7), (2, 4, 2, 1, 13),
                                         (4, 2, 2, 2, 3), (2, 1, 4, 1, 3), (1, 2, 4, 1, 6)])
@pytest.mark.parametrize("M", [4, 16])
def test_lockstep_narrow_slabs(cuda, KG, T, U, S, SW, M):
    P = O.Problem(O.INT4, M, 2048, 1000, 128, O.F16, seed=3050 + M + SW)
    D = DeviceProblem(P)
    with decode_env(KERNEL=1, LS_KG=KG, LS_T=T, LS_U=U, LS_S=S, LS_SW=SW):
        y = D.run()
    check(y, P.reference(), O.F16, f"KG={KG} T={T} U={U} S={S} SW={SW} M={M}", P)


@pytest.mark.parametrize("fmt,xdt", [(O.INT4, O.BF16), (O.TERNARY2, O.F16), (O.TERNARY2, O.BF16)])
@pytest.mark.parametrize("KG,T,U,S", [(2, 2, 2, 1), (2, 2, 2, 3), (4, 2, 3, 2), (2, 1, 4, 1), (1, 2, 4, 2)])
def test_lockstep_formats(cuda, fmt, xdt, KG, T, U, S):
    # group 256: one scale row serves two k-blocks.
    P = O.Problem(fmt, 9, 1536, 700, 256, xdt, seed=3100)
    D = DeviceProblem(P)
    with decode_env(KERNEL=1, LS_KG=KG, LS_T=T, LS_U=U, LS_S=S):
        y = D.run()
    check(y, P.reference(), xdt, f"fmt={fmt} KG={KG} T={T} U={U} S={S}", P)


@pytest.mark.parametrize("S,SW", [(1, 0), (3, 0), (1, 7), (2, 5)])
def test_lockstep_fused(cuda, S, SW):
    # Slabs never straddle segments; each segment's last slab is partial.
    Ns, K, M = [600, 130, 1000], 1024, 6
    probs = [O.Problem(O.INT4, M, K, n, 128, O.F16, seed=3200 + i) for i, n in enumerate(Ns)]
    for p in probs[1:]:
        p.X = probs[0].X
    devs = [DeviceProblem(p) for p in probs]
    with decode_env(KERNEL=1, LS_S=S, **({"LS_SW": SW} if SW else {})):
        outs = hq.gemm_fused(O.INT4, devs[0].X, [(d.Wp, d.S, d.P.N) for d in devs])
    for d, y in zip(devs, outs):
        check(y, d.P.reference(), O.F16, f"lockstep fused S={S} SW={SW} N={d.P.N}", d.P)


@pytest.mark.parametrize("M", [4, 16])
def test_lockstep_matches_per_wavefront(cuda, M):
    # The two decode kernels compute the same values up to fp32 summation order.
    P = O.Problem(O.INT4, M, 5120, 5120, 128, O.F16, seed=3300 + M)
    D = DeviceProblem(P)
    with decode_env(KERNEL=1):
        y1 = D.run()
    with decode_env(KERNEL=0):
        y0 = D.run()
    assert O.normwise_error(to_host_f32(y1), to_host_f32(y0)) <= OUT_TOL[O.F16]
    check(y1, P.reference(threads=16), O.F16, f"lockstep M={M}")


# ---------------------------------------------------------------- X-resident decode kernel
class xr_env(decode_env):
    """Force the X-resident decode kernel (activation rows in LDS) and its tiling for a block:
    slab width T, wavefronts WK (splitting the slab's k-blocks), ring depth U, pieces S, slab
    count G (slabs of fewer than T tiles), slab groups SG per workgroup."""

    def __init__(self, **kv):
        self.kv = {f"HQ_XR_{k}": str(v) for k, v in kv.items()}
        self.kv["HQ_DECODE_KERNEL"] = "2"


# (T, WK, U): every instantiated (slab width, ring depth); one wavefront, wavefront counts that
# do not divide the 16 k-blocks, and 16 wavefronts of one k-block each.
XR_CFGS = [(1, 1, 4), (1, 3, 6), (1, 16, 4), (2, 4, 3), (2, 7, 4), (2, 16, 3), (4, 5, 2), (4, 16, 2), (8, 4, 2),
           (8, 8, 2)]


@pytest.mark.parametrize("T,WK,U", XR_CFGS)
@pytest.mark.parametrize("M", [1, 6, 16])
def test_xr_configs_int4(cuda, T, WK, U, M):
    # K = 2048 (16 k-blocks), N = 1000 (63 tiles: the last slab is partial for every width).
    P = O.Problem(O.INT4, M, 2048, 1000, 128, O.F16, seed=3400 + M)
    D = DeviceProblem(P)
    with xr_env(T=T, WK=WK, U=U):
        assert hq.describe(O.INT4, O.F16, M, 2048, 1000).startswith(f"hq_decode_xr_kernel<int4,f16,T={T},U={U}>")
        y = D.run()
        y2 = D.run()
    assert torch_equal(y, y2)  # fixed summation order: bit-identical from run to run
    check(y, P.reference(), O.F16, f"xr T={T} WK={WK} U={U} M={M}", P)


@pytest.mark.parametrize("fmt,xdt", [(O.INT4, O.BF16), (O.TERNARY2, O.F16), (O.TERNARY2, O.BF16)])
@pytest.mark.parametrize("T,WK,U", [(1, 8, 4), (2, 8, 3), (4, 4, 2), (8, 8, 2)])
def test_xr_formats(cuda, fmt, xdt, T, WK, U):
    # group 256: one scale row serves two k-blocks.
    P = O.Problem(fmt, 9, 1536, 700, 256, xdt, seed=3450)
    D = DeviceProblem(P)
    with xr_env(T=T, WK=WK, U=U):
        assert "hq_decode_xr_kernel" in hq.describe(fmt, xdt, 9, 1536, 700, group=256)
        y = D.run()
    check(y, P.reference(), xdt, f"xr fmt={fmt} T={T} WK={WK} U={U}", P)


@pytest.mark.parametrize("T", [2, 8])
def test_xr_fused(cuda, T):
    # Slabs never straddle segments; each segment's last slab is partial.
    Ns, K, M = [600, 130, 1000], 1024, 5
    probs = [O.Problem(O.INT4, M, K, n, 128, O.F16, seed=3500 + i) for i, n in enumerate(Ns)]
    for p in probs[1:]:
        p.X = probs[0].X
    devs = [DeviceProblem(p) for p in probs]
    with xr_env(T=T, WK=4):
        outs = hq.gemm_fused(O.INT4, devs[0].X, [(d.Wp, d.S, d.P.N) for d in devs])
    for d, y in zip(devs, outs):
        check(y, d.P.reference(), O.F16, f"xr fused T={T} N={d.P.N}", d.P)


@pytest.mark.parametrize("fmt,xdt", [(O.INT4, O.F16), (O.TERNARY2, O.BF16)])
@pytest.mark.parametrize("T,G,WK", [(4, 30, 4), (8, 20, 8), (2, 50, 8)])
def test_xr_variable_width_slabs(cuda, fmt, xdt, T, G, WK):
    # A slab count above ceil(tiles / T) (HQ_XR_G) cuts slabs of fewer than T tiles, of two
    # widths: 63 tiles in 30 slabs of 2-3 tiles (T = 4), 20 of 3-4 (T = 8), 50 of 1-2 (T = 2).
    # The missing tiles' loads read nothing and their columns are never stored.
    M, K, N = 5, 2048, 1000
    P = O.Problem(fmt, M, K, N, 128, xdt, seed=3520 + T)
    D = DeviceProblem(P)
    with xr_env(T=T, G=G, WK=WK):
        desc = hq.describe(fmt, xdt, M, K, N)
        assert desc.startswith("hq_decode_xr_kernel<") and f",T={T}," in desc and f"workgroups={G} slabs" in desc, desc
        y = D.run()
    check(y, P.reference(), xdt, f"xr variable slabs T={T} G={G}", P)


# Slab groups: SG groups of WK wavefronts per workgroup over one copy of the activation rows,
# group h of workgroup b streaming slab b + h * gridDim.x; a ragged last workgroup (an odd slab
# count) has a group with no slab, which loads and stores nothing.
@pytest.mark.parametrize("fmt,xdt", [(O.INT4, O.F16), (O.TERNARY2, O.BF16), (O.INT4, O.BF16)])
@pytest.mark.parametrize("WK,SG,G", [(4, 2, 0), (4, 2, 31), (2, 4, 33), (4, 3, 0), (8, 2, 0), (1, 4, 0)])
@pytest.mark.parametrize("M", [1, 8, 16])
def test_xr_slab_groups(cuda, fmt, xdt, WK, SG, G, M):
    import torch

    K, N = 2048, 1000  # 63 tiles: 16 slabs of 4 tiles, the last one of 3
    P = O.Problem(fmt, M, K, N, 128, xdt, seed=3580 + 7 * M + SG + G)
    D = DeviceProblem(P)
    kw = dict(T=4, WK=WK, SG=SG, S=1, **({"G": G} if G else {}))
    with xr_env(**kw):
        desc = hq.describe(fmt, xdt, M, K, N)
        assert desc.startswith("hq_decode_xr_kernel<") and f",T=4,U=2,SG={SG}>" in desc, desc
        y = D.run()
        y2 = D.run()
    assert torch.equal(y, y2)
    check(y, P.reference(), xdt, f"xr slab groups {kw} M={M}", P)


def test_xr_slab_groups_fused(cuda):
    # The groups of one workgroup may stream slabs of different segments.
    Ns, K, M = [600, 130, 1000], 1024, 5
    probs = [O.Problem(O.INT4, M, K, n, 128, O.F16, seed=3590 + i) for i, n in enumerate(Ns)]
    for p in probs[1:]:
        p.X = probs[0].X
    devs = [DeviceProblem(p) for p in probs]
    for kw in (dict(T=4, WK=4, SG=2, S=1), dict(T=4, WK=4, SG=3, S=1, G=41)):
        with xr_env(**kw):
            outs = hq.gemm_fused(O.INT4, devs[0].X, [(d.Wp, d.S, d.P.N) for d in devs])
        for d, y in zip(devs, outs):
            check(y, d.P.reference(), O.F16, f"xr slab groups fused {kw} N={d.P.N}", d.P)


@pytest.mark.parametrize("M,K", [(16, 5120), (8, 5120), (3, 5120), (2, 27648), (1, 27648)])
def test_xr_lds_limits(cuda, M, K):
    # Whole-K plans whose activation rows fill the LDS (16 x 5120 halves = 160 KiB), half of
    # it, or hold the longest K (27648) for one and two rows.
    N = 1000
    P = O.Problem(O.INT4, M, K, N, 128, O.F16, seed=3550 + M)
    D = DeviceProblem(P)
    with xr_env(T=2, WK=8, S=1):
        desc = hq.describe(O.INT4, O.F16, M, K, N)
        assert desc.startswith("hq_decode_xr_kernel<int4,f16,") and f"lds={M * K * 2}" in desc, desc
        y = D.run()
    check(y, P.reference(threads=16), O.F16, f"xr lds M={M} K={K}", P)


@pytest.mark.parametrize("fmt,xdt,M,K,N", [(O.TERNARY2, O.F16, 1, 5120, 34816), (O.INT4, O.BF16, 2, 4096, 40960)])
def test_xr_spilled_4tile_slabs_take_4wave_2tile_slabs(cuda, fmt, xdt, M, K, N):
    # More 4-tile slabs than one round holds, at one or two rows: the planner takes 2-tile
    # slabs of four wavefronts (one round on MI355X by the occupancy query).
    P = O.Problem(fmt, M, K, N, 128, xdt, seed=3650 + M)
    desc = hq.describe(fmt, xdt, M, K, N)
    assert desc.startswith("hq_decode_xr_kernel<") and ",T=2,U=3>" in desc and "x 4 wavefronts" in desc, desc
    check(DeviceProblem(P).run(), P.reference(threads=16), xdt, f"4-wave 2-tile slabs M={M} N={N}", P)


@pytest.mark.parametrize("fmt,xdt,M,N", [(O.INT4, O.F16, 1, 27648), (O.INT4, O.F16, 8, 27648), (O.TERNARY2, O.BF16, 4, 34816)])
def test_xr_whole_4tile_slabs_take_4_wavefronts(cuda, fmt, xdt, M, N):
    # Whole 4-tile slabs at up to eight rows whose grid still fits on the CUs in one round run
    # with four wavefronts per slab (one per SIMD) instead of eight: the decode sweep's 5120 x
    # 27648 (int4: two such slabs per workgroup) and the decoder's fused gate||up width (three
    # per workgroup at four rows).
    K = 5120
    desc = hq.describe(fmt, xdt, M, K, N)
    assert desc.startswith("hq_decode_xr_kernel<") and ",T=4," in desc and "x 1 pieces x 4 wavefronts" in desc, desc
    assert (",SG=2>" in desc) == (fmt == O.INT4 and N == 27648), desc
    assert (",SG=3>" in desc) == (N == 34816), desc
    P = O.Problem(fmt, M, K, N, 128, xdt, seed=3660 + M)
    check(DeviceProblem(P).run(), P.reference(threads=16), xdt, f"4-wave 4-tile slabs M={M} N={N}", P)


@pytest.mark.parametrize("fmt,xdt,M,K,N", [(O.INT4, O.F16, 9, 5120, 17408), (O.INT4, O.BF16, 1, 4096, 22528),
                                           (O.TERNARY2, O.BF16, 12, 4096, 18432), (O.INT4, O.F16, 16, 5120, 20480)])
def test_xr_slab_pairs_just_past_one_slab_per_cu(cuda, fmt, xdt, M, K, N):
    # 272-352 whole 4-tile slabs (just past one per CU): pairs per workgroup (asserted on
    # 256-CU devices), the grid one round; against the oracle.
    import torch

    desc = hq.describe(fmt, xdt, M, K, N)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert desc.startswith("hq_decode_xr_kernel<") and ",SG=2>" in desc, desc
    P = O.Problem(fmt, M, K, N, 128, xdt, seed=4300 + M)
    check(DeviceProblem(P).run(), P.reference(threads=16), xdt, f"pairs M={M} K={K} N={N}: {desc}", P)


@pytest.mark.parametrize("fmt,xdt,M,K,N,sg", [(O.INT4, O.F16, 4, 5120, 34816, 3), (O.TERNARY2, O.BF16, 16, 4096, 40960, 3),
                                              (O.INT4, O.BF16, 12, 4096, 49280, 4), (O.TERNARY2, O.F16, 1, 5120, 55296, 4),
                                              (O.INT4, O.F16, 16, 4096, 57344, 4)])
def test_xr_slab_groups_default_plan(cuda, fmt, xdt, M, K, N, sg):
    # 513-1024 whole 4-tile slabs: triples and quads of slabs per workgroup (asserted on 256-CU
    # devices), the last workgroup ragged where the groups do not divide the slabs (544, 640
    # and 770 slabs); against the oracle.
    import torch

    desc = hq.describe(fmt, xdt, M, K, N)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        slabs = N // 64
        assert f",T=4,U=2,SG={sg}> workgroups={(slabs + sg - 1) // sg} of {sg} slabs" in desc, desc
    P = O.Problem(fmt, M, K, N, 128, xdt, seed=4400 + M)
    check(DeviceProblem(P).run(), P.reference(threads=16), xdt, f"slab groups M={M} K={K} N={N}: {desc}", P)


@pytest.mark.parametrize("fmt,xdt,M,N", [(O.TERNARY2, O.F16, 12, 14336), (O.INT4, O.BF16, 16, 14336),
                                         (O.TERNARY2, O.BF16, 9, 16384), (O.INT4, O.F16, 16, 27648)])
def test_xr_wide_rows_default_plan(cuda, fmt, xdt, M, N):
    # Wide weights at more than eight rows, as the planner takes them: one round of 4-tile
    # X-resident slabs (the decoder's fused QKV and SSM projections), pairs of 4-tile slabs per
    # workgroup when single slabs would take more than one round (5120 x 27648: 432 slabs).
    K = 5120
    P = O.Problem(fmt, M, K, N, 128, xdt, seed=3600 + M)
    desc = hq.describe(fmt, xdt, M, K, N)
    assert desc.startswith("hq_decode_xr_kernel<") and ",T=4," in desc and "x 1 pieces" in desc, desc
    assert (",SG=2>" in desc) == (N == 27648), desc
    check(DeviceProblem(P).run(), P.reference(threads=16), xdt, f"wide rows {desc[:40]} M={M} N={N}", P)


# K pieces per slab (S): even and uneven splits of 16 k-blocks, one k-block per piece, and
# pieces that leave some wavefronts without k-blocks; the last of a slab's workgroups sums
# the partials in piece order (bit-identical from run to run) and leaves its counter at zero.
@pytest.mark.parametrize("T,WK,U,S", [(2, 8, 3, 2), (2, 4, 4, 3), (4, 8, 2, 5), (8, 4, 2, 16), (1, 3, 4, 7),
                                      (8, 8, 2, 6)])
@pytest.mark.parametrize("M", [1, 7, 16])
def test_xr_pieces(cuda, T, WK, U, S, M):
    import torch

    P = O.Problem(O.INT4, M, 2048, 1000, 128, O.F16, seed=3700 + M)
    D = DeviceProblem(P)
    with xr_env(T=T, WK=WK, U=U, S=S):
        desc = hq.describe(O.INT4, O.F16, M, 2048, 1000)
        assert desc.startswith(f"hq_decode_xr_kernel<int4,f16,T={T},U={U}>") and f"x {S} pieces" in desc, desc
        need = hq.workspace_bytes(O.INT4, M, 2048, 1000)
        assert need > 0
        ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
        y = hq.gemm(O.INT4, D.X, D.Wp, D.S, 1000, workspace=ws)
        y2 = hq.gemm(O.INT4, D.X, D.Wp, D.S, 1000, workspace=ws)
        y3 = D.run()  # the library's own workspace
    assert torch_equal(y, y2) and torch_equal(y, y3)
    torch.cuda.synchronize()
    assert int(ws[:4 * 64].view(torch.int32).abs().sum().item()) == 0  # counters back at zero
    check(y, P.reference(), O.F16, f"xr pieces T={T} WK={WK} U={U} S={S} M={M}", P)


@pytest.mark.parametrize("fmt,xdt", [(O.TERNARY2, O.BF16), (O.INT4, O.BF16)])
def test_xr_pieces_fused(cuda, fmt, xdt):
    Ns, K, M = [600, 130, 1000], 1536, 9
    probs = [O.Problem(fmt, M, K, n, 256, xdt, seed=3750 + i) for i, n in enumerate(Ns)]
    for p in probs[1:]:
        p.X = probs[0].X
    devs = [DeviceProblem(p) for p in probs]
    with xr_env(T=4, WK=8, S=5):
        outs = hq.gemm_fused(fmt, devs[0].X, [(d.Wp, d.S, d.P.N) for d in devs], group=256)
    for d, y in zip(devs, outs):
        check(y, d.P.reference(), xdt, f"xr pieces fused N={d.P.N}", d.P)


@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_xr_pieces_default_plans(cuda, M):
    # K = 27648, N = 1000: 32 whole slabs would leave most CUs idle (and from M = 3 on the rows
    # of all of K do not fit in LDS); the planner cuts K.
    K, N = 27648, 1000
    desc = hq.describe(O.INT4, O.F16, M, K, N)
    assert desc.startswith("hq_decode_xr_kernel<int4,f16,") and "x 1 pieces" not in desc, desc
    P = O.Problem(O.INT4, M, K, N, 128, O.F16, seed=3800 + M)
    D = DeviceProblem(P)
    check(D.run(), P.reference(threads=16), O.F16, f"xr default pieces M={M}", P)


@pytest.mark.parametrize("fmt,xdt,M,K,N,plan", [
    (O.INT4, O.F16, 1, 5120, 1024, "T=1,U=4> workgroups=64 slabs x 1 pieces"),
    (O.INT4, O.F16, 8, 5120, 1000, "T=1,U=4> workgroups=63 slabs x 1 pieces"),
    (O.TERNARY2, O.BF16, 16, 5120, 1024, "T=1,U=4> workgroups=64 slabs x 1 pieces"),
    (O.INT4, O.BF16, 16, 8192, 2048, "T=1,U=4> workgroups=128 slabs x 2 pieces"),
    (O.INT4, O.F16, 1, 27648, 1024, "T=1,U=4> workgroups=64 slabs x 4 pieces"),
    (O.TERNARY2, O.F16, 8, 27648, 520, "T=1,U=4> workgroups=33 slabs x 4 pieces"),
    (O.INT4, O.F16, 16, 14336, 1024, "T=1,U=4> workgroups=64 slabs x 3 pieces"),
    (O.INT4, O.F16, 1, 4096, 14336, "T=4,U=2> workgroups=224 slabs x 1 pieces x 8 wavefronts"),
    (O.TERNARY2, O.BF16, 4, 4096, 11008, "T=4,U=2> workgroups=172 slabs x 1 pieces x 8 wavefronts"),
    (O.TERNARY2, O.BF16, 1, 27648, 5120, "T=4,U=2> workgroups=80 slabs x 3 pieces x 8 wavefronts"),
    (O.TERNARY2, O.F16, 2, 27648, 5120, "T=4,U=2> workgroups=80 slabs x 3 pieces x 8 wavefronts"),
])
def test_xr_default_plans_by_tile_count(cuda, fmt, xdt, M, K, N, plan):
    # Few tiles (GQA key/value widths): one-tile slabs, whole or in K pieces; 4-tile slabs one
    # to a CU where 2-tile slabs would take two; ternary over a long K in K pieces at one or two
    # rows (plans asserted on 256-CU devices).
    import torch

    desc = hq.describe(fmt, xdt, M, K, N)
    assert desc.startswith("hq_decode_xr_kernel<"), desc
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert plan in desc, desc
    P = O.Problem(fmt, M, K, N, 128, xdt, seed=4100 + M + K // 1024)
    D = DeviceProblem(P)
    y = D.run()
    assert torch_equal(y, D.run())
    check(y, P.reference(threads=16), xdt, f"default plan M={M} K={K} N={N}: {desc}", P)


@pytest.mark.parametrize("M", [1, 4, 16])
def test_xr_matches_other_decode_kernels(cuda, M):
    # The three decode kernels compute the same values up to fp32 summation order.
    P = O.Problem(O.INT4, M, 5120, 5120, 128, O.F16, seed=3600 + M)
    D = DeviceProblem(P)
    assert hq.describe(O.INT4, O.F16, M, 5120, 5120).startswith("hq_decode_xr_kernel")
    y2 = D.run()
    with decode_env(KERNEL=1):
        y1 = D.run()
    with decode_env(KERNEL=0):
        y0 = D.run()
    assert O.normwise_error(to_host_f32(y2), to_host_f32(y1)) <= OUT_TOL[O.F16]
    assert O.normwise_error(to_host_f32(y2), to_host_f32(y0)) <= OUT_TOL[O.F16]
    check(y2, P.reference(threads=16), O.F16, f"xr M={M}")


class prefill_env(decode_env):
    """Force the prefill kernel (also for M <= 80, which the lockstep kernel takes by
    default) and its tiling for a block: WM (tile height 128 or 256 rows), SK=0 (no
    stream-K), TAIL=0 (no half-height tail launch), PSK (stream-K workgroups)."""

    def __init__(self, **kv):
        self.kv = {f"HQ_PREFILL_{k}": str(v) for k, v in kv.items()}
        self.kv["HQ_DECODE_MAX_M"] = "16"


def normwise_between(a, b):
    a, b = to_host_f32(a).astype(np.float64), to_host_f32(b).astype(np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


# Prefill grids smaller than half the workgroup slots split their tiles along K (stream-K,
# by default s ways) and sum them in a last-arriver fix-up. That must agree with
# whole-tile execution up to fp32 summation order (two output ulps of the largest value,
# normwise) and be bit-reproducible.
@pytest.mark.parametrize("fmt,xdt,M,K,N,psk", [
    (O.TERNARY2, O.BF16, 512, 5120, 27648, 432),  # all 216 tiles split 2 ways (forced)
    (O.INT4, O.F16, 256, 27648, 5120, 0),         # 80 64-row tiles split 6 ways (short pieces)
    (O.INT4, O.F16, 1024, 27648, 5120, 0),        # 160 128-row tiles split 3 ways (72 k-blocks each)
    (O.INT4, O.BF16, 40, 4096, 4096, 0),          # 64-row tiles, 16 tiles split 8 ways
    (O.TERNARY2, O.F16, 200, 2048, 3000, 0),
    (O.INT4, O.F16, 129, 1024, 700, 0),
    (O.INT4, O.F16, 129, 1024, 700, 5),           # ranges straddling tiles
])
def test_prefill_stream_k_equals_whole_tiles(cuda, fmt, xdt, M, K, N, psk):
    P = O.Problem(fmt, M, K, N, 128, xdt, seed=2600 + M)
    D = DeviceProblem(P)
    with prefill_env(PSK=psk):
        y = D.run()
        assert torch_equal(y, D.run())
    with prefill_env(SK=0, TAIL=0):
        y_whole = D.run()
    tol = 2 * (2.0**-11 if xdt == O.F16 else 2.0**-8)
    assert normwise_between(y, y_whole) <= tol
    if M * K * N <= 4e9:
        check(y, P.reference(), xdt, f"stream-K fmt={fmt} M={M} K={K} N={N}", P)
    else:
        rows = np.sort(np.random.default_rng(M).choice(M, size=16, replace=False))
        err = O.normwise_error(to_host_f32(y)[rows], P.reference(rows=rows, threads=16))
        assert err <= OUT_TOL[xdt]


# 256-row tiles (one workgroup per CU, on request): a part-empty last round of whole tiles
# runs the last column blocks as a second launch of half-height tiles. Each output element
# is the same fp32 chain in the same k order, so the result equals whole-tile execution bit
# for bit, and both match the default 128-row tiling. The fused case cuts a segment.
@pytest.mark.parametrize("fmt,xdt,M,Ns", [
    (O.INT4, O.F16, 2048, [27648]),         # 864 tiles: the last 12 of 108 blocks as 128-row tiles
    (O.TERNARY2, O.BF16, 3072, [27648]),
    (O.INT4, O.BF16, 2048, [26648, 1000]),  # 109 blocks: the tail spans both segments
])
def test_prefill_tail_equals_whole_tiles(cuda, fmt, xdt, M, Ns):
    K = 1024
    probs = [O.Problem(fmt, M, K, n, 128, xdt, seed=2650 + i) for i, n in enumerate(Ns)]
    for p in probs[1:]:
        p.X = probs[0].X
    devs = [DeviceProblem(p) for p in probs]
    segs = [(d.Wp, d.S, d.P.N) for d in devs]
    with prefill_env(WM=2):
        outs = hq.gemm_fused(fmt, devs[0].X, segs)
    with prefill_env(WM=2, SK=0, TAIL=0):
        whole = hq.gemm_fused(fmt, devs[0].X, segs)
    default = hq.gemm_fused(fmt, devs[0].X, segs)
    rows = np.sort(np.random.default_rng(M).choice(M, size=8, replace=False))
    for d, y, w, y128 in zip(devs, outs, whole, default):
        assert torch_equal(y, w)
        assert torch_equal(y, y128)
        err = O.normwise_error(to_host_f32(y)[rows], d.P.reference(rows=rows, threads=16))
        assert err <= OUT_TOL[xdt]


# The K split inside the workgroup (KS=2: two halves of four wavefronts, each over half of the
# tile's k-blocks, summed in LDS) against whole tiles without it: the same values up to fp32
# summation order, bit-reproducible, and the oracle's. Forced on grids of several rounds,
# ragged M and N, fused segments, every format and dtype; by default it takes one-round grids
# of 128-row tiles covering at least three quarters of the CUs (fused QKV at M = 1024).
@pytest.mark.parametrize("fmt,xdt,M,K,N", [
    (O.INT4, O.F16, 300, 2048, 1000),
    (O.INT4, O.BF16, 129, 1024, 4000),
    (O.TERNARY2, O.F16, 200, 4096, 700),
    (O.TERNARY2, O.BF16, 1000, 1024, 2600),
    (O.INT4, O.F16, 2048, 5120, 27648),
])
def test_prefill_k_split_in_workgroup(cuda, fmt, xdt, M, K, N):
    P = O.Problem(fmt, M, K, N, 128, xdt, seed=2750 + M)
    D = DeviceProblem(P)
    with prefill_env(KS=2, WM=1, SK=0, TAIL=0):  # 128-row tiles (small grids would take 64)
        assert "k-split in workgroup" in hq.describe(fmt, xdt, M, K, N)
        y = D.run()
        assert torch_equal(y, D.run())
    with prefill_env(KS=1, WM=1, SK=0, TAIL=0):
        y1 = D.run()
    tol = 2 * (2.0**-11 if xdt == O.F16 else 2.0**-8)
    assert normwise_between(y, y1) <= tol
    if M * K * N <= 4e9:
        check(y, P.reference(), xdt, f"k-split fmt={fmt} M={M} K={K} N={N}", P)
    else:
        rows = np.sort(np.random.default_rng(M).choice(M, size=16, replace=False))
        assert O.normwise_error(to_host_f32(y)[rows], P.reference(rows=rows, threads=16)) <= OUT_TOL[xdt]


def test_prefill_k_split_fused_default_plan(cuda):
    # Fused QKV shape of the split-fuse step (M = 1024, N = 5120 | 1024 | 1024): 224 256-column
    # tiles would take the K split; with fp16 activations 448 128-column tiles run by default
    # (on a 256-CU part), the K split itself forced here.
    Ns, K, M = [5120, 1024, 1024], 5120, 1024
    probs = [O.Problem(O.INT4, M, K, n, 128, O.F16, seed=2760 + i) for i, n in enumerate(Ns)]
    for p in probs[1:]:
        p.X = probs[0].X
    devs = [DeviceProblem(p) for p in probs]
    segs = [(d.Wp, d.S, d.P.N) for d in devs]
    with prefill_env(KS=2, WM=1):
        outs = hq.gemm_fused(O.INT4, devs[0].X, segs)
    with prefill_env(KS=1, SK=0, TAIL=0):
        ref_outs = hq.gemm_fused(O.INT4, devs[0].X, segs)
    rows = np.sort(np.random.default_rng(5).choice(M, size=12, replace=False))
    for d, y, y1 in zip(devs, outs, ref_outs):
        assert normwise_between(y, y1) <= 2 * 2.0**-11
        assert O.normwise_error(to_host_f32(y)[rows], d.P.reference(rows=rows, threads=16)) <= OUT_TOL[O.F16]


# 128-row x 128-column whole tiles (four wavefronts of two column tiles each) against the
# 256-column tiles: the same values up to fp32 summation order (each output's k order is the
# same, so in practice equal), bit-reproducible, and the oracle's. Ragged M and N (wavefronts
# past N, partial last bands), the column tiles of fused segments, every format and dtype.
@pytest.mark.parametrize("fmt,xdt,M,K,N", [
    (O.INT4, O.F16, 300, 2048, 1000),
    (O.INT4, O.BF16, 129, 1024, 4000),
    (O.TERNARY2, O.F16, 200, 4096, 720),
    (O.TERNARY2, O.BF16, 1000, 1024, 2600),
    (O.INT4, O.F16, 1024, 5120, 7168),
])
def test_prefill_128_column_tiles(cuda, fmt, xdt, M, K, N):
    P = O.Problem(fmt, M, K, N, 128, xdt, seed=2790 + M)
    D = DeviceProblem(P)
    with prefill_env(TW=2, WM=1, SK=0, TAIL=0):
        desc = hq.describe(fmt, xdt, M, K, N)
        assert "128-row 128-column tiles" in desc, desc
        y = D.run()
        assert torch_equal(y, D.run())
    with prefill_env(KS=1, WM=1, SK=0, TAIL=0):
        y1 = D.run()
    assert normwise_between(y, y1) <= 2 * (2.0**-11 if xdt == O.F16 else 2.0**-8)
    if M * K * N <= 4e9:
        check(y, P.reference(), xdt, f"128-column tiles fmt={fmt} M={M} K={K} N={N}", P)
    else:
        rows = np.sort(np.random.default_rng(M).choice(M, size=16, replace=False))
        assert O.normwise_error(to_host_f32(y)[rows], P.reference(rows=rows, threads=16)) <= OUT_TOL[xdt]


def test_prefill_128_column_tiles_fused(cuda):
    # Fused segments whose widths are not multiples of 128 columns (each segment starts a new
    # column block).
    Ns, K, M = [600, 130, 1000], 1024, 300
    probs = [O.Problem(O.INT4, M, K, n, 128, O.F16, seed=2795 + i) for i, n in enumerate(Ns)]
    for p in probs[1:]:
        p.X = probs[0].X
    devs = [DeviceProblem(p) for p in probs]
    with prefill_env(TW=2, WM=1, SK=0, TAIL=0):
        outs = hq.gemm_fused(O.INT4, devs[0].X, [(d.Wp, d.S, d.P.N) for d in devs])
    for d, y in zip(devs, outs):
        check(y, d.P.reference(), O.F16, f"128-column tiles fused N={d.P.N}", d.P)


# The default plans that take 128-column tiles (asserted on 256-CU devices) and neighbours
# that keep 256-column tiles; rows at every band boundary against the oracle.
@pytest.mark.parametrize("fmt,xdt,M,K,N,tw2", [
    (O.INT4, O.BF16, 768, 5120, 7168, True),       # in place of 336 64-row tiles
    (O.TERNARY2, O.F16, 384, 4096, 11008, True),    # in place of 258 64-row tiles
    (O.INT4, O.F16, 704, 5120, 7168, True),         # 128-row bands 64 rows taller than 64-row ones
    (O.INT4, O.F16, 192, 5120, 36864, False),       # 432 64-row tiles stay (576 128-column tiles)
    (O.INT4, O.F16, 128, 5120, 27648, True),        # one band of 128 rows in place of two of 64
    (O.TERNARY2, O.F16, 128, 5120, 27648, False),   # ... except ternary fp16 at 216 tiles
    (O.TERNARY2, O.F16, 112, 5120, 34816, True),    # ... which takes them at 272
    (O.INT4, O.BF16, 96, 5120, 34816, True),        # M = 81..127: one band of 128 rows
    (O.INT4, O.F16, 96, 5120, 14336, False),        # stream-K of 64-row tiles stays
    (O.TERNARY2, O.BF16, 512, 5120, 17408, True),   # bf16 in place of 272 128-row tiles
    (O.INT4, O.F16, 512, 5120, 17408, False),       # fp16 keeps them
    (O.TERNARY2, O.F16, 1024, 5120, 7168, True),    # fp16 in place of the K split
    (O.TERNARY2, O.BF16, 1024, 5120, 7168, False),  # bf16 keeps it
    (O.INT4, O.BF16, 768, 5120, 12288, True),       # bf16 in place of 288 128-row tiles
    (O.INT4, O.F16, 1024, 27648, 5120, False),      # stream-K over a long K stays
])
def test_prefill_128_column_tiles_default_plan(cuda, fmt, xdt, M, K, N, tw2):
    import torch

    desc = hq.describe(fmt, xdt, M, K, N)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert ("128-column" in desc) == tw2, desc
    P = O.Problem(fmt, M, K, N, 128, xdt, seed=4250 + M)
    y = to_host_f32(DeviceProblem(P).run())
    rows = np.array(sorted(r for r in {0, 1, 63, 64, 127, 128, 129, M // 2, M - 2, M - 1} if r < M))
    ref = P.reference(rows=rows, threads=16)
    assert O.normwise_error(y[rows], ref) <= OUT_TOL[xdt], desc
    elementwise_bound_check(y[rows], ref, P, rows=rows)


# Forced stream-K grids on 15 tiles of 64 rows x 256 columns, K = 1024 (8 k-blocks):
# 16 workgroups give ranges of 8 units aligned to tiles (whole-tile pieces inside the
# stream-K part), 17 and 40 give ranges that straddle tiles, 119 gives 1-unit ranges.
@pytest.mark.parametrize("psk", [16, 17, 40, 119])
def test_prefill_stream_k_grids(cuda, psk):
    P = O.Problem(O.INT4, 17, 1024, 3840, 128, O.F16, seed=2700 + psk)
    D = DeviceProblem(P)
    with prefill_env(PSK=psk):
        y = D.run()
    check(y, P.reference(), O.F16, f"psk={psk}", P)


def test_prefill_stream_k_fused(cuda):
    Ns, K, M = [1000, 300, 2600], 2048, 300
    probs = [O.Problem(O.TERNARY2, M, K, n, 128, O.F16, seed=2800 + i) for i, n in enumerate(Ns)]
    for p in probs[1:]:
        p.X = probs[0].X
    devs = [DeviceProblem(p) for p in probs]
    for psk in (0, 37):
        with prefill_env(PSK=psk):
            outs = hq.gemm_fused(O.TERNARY2, devs[0].X, [(d.Wp, d.S, d.P.N) for d in devs])
        for d, y in zip(devs, outs):
            check(y, d.P.reference(), O.F16, f"fused stream-K psk={psk} N={d.P.N}", d.P)


def test_prefill_caller_workspace_reused(cuda):
    import torch

    # Two stream-K prefill calls (N = 256: 16 and 5 output tiles) share one caller workspace of
    # the larger of their sizes.
    K, N = 5120, 256
    need = max(hq.workspace_bytes(O.INT4, M, K, N) for M in (2048, 300))
    assert need > 0
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    P = O.Problem(O.INT4, 2048, K, N, 128, O.F16, seed=2900)
    D = DeviceProblem(P)
    y_int = D.run()
    assert torch_equal(hq.gemm(O.INT4, D.X, D.Wp, D.S, N, workspace=ws), y_int)
    X300 = D.X[:300].contiguous()
    assert torch_equal(hq.gemm(O.INT4, X300, D.Wp, D.S, N, workspace=ws), D.run(X=X300))
    torch.cuda.synchronize()
    assert int(ws[:65536].view(torch.int32).abs().sum().item()) == 0  # counters left at zero


# ---------------------------------------------------------------- lockstep kernel, 17 <= M <= 80
# Two to five 16-row tiles per workgroup share each dequantised weight fragment (a
# split-fuse step of 16 decode tokens and a 64-token prefill chunk is one weight stream).
@pytest.mark.parametrize("M", [17, 31, 32, 48, 63, 64, 65, 79, 80])
def test_lockstep_row_tiles_int4(cuda, M):
    P = O.Problem(O.INT4, M, 2048, 1000, 128, O.F16, seed=3400 + M)
    D = DeviceProblem(P)
    y = D.run()
    assert torch_equal(y, D.run())
    check(y, P.reference(), O.F16, f"row tiles M={M}", P)


@pytest.mark.parametrize("fmt,xdt,M", [(O.INT4, O.BF16, 40), (O.TERNARY2, O.F16, 33), (O.TERNARY2, O.BF16, 80)])
def test_lockstep_row_tiles_formats(cuda, fmt, xdt, M):
    P = O.Problem(fmt, M, 1536, 700, 256, xdt, seed=3500 + M)
    check(DeviceProblem(P).run(), P.reference(), xdt, f"row tiles fmt={fmt} M={M}", P)


@pytest.mark.parametrize("M,S", [(24, 3), (80, 5), (50, 2)])
def test_lockstep_row_tiles_split(cuda, M, S):
    # Slabs cut along K: every row tile's partials go through the fix-up.
    P = O.Problem(O.INT4, M, 4096, 640, 128, O.F16, seed=3600 + M)
    D = DeviceProblem(P)
    with decode_env(LS_S=S):
        y = D.run()
        assert torch_equal(y, D.run())
    check(y, P.reference(), O.F16, f"row tiles split S={S} M={M}", P)


@pytest.mark.parametrize("fmt,xdt,M", [(O.INT4, O.F16, 40), (O.INT4, O.BF16, 80), (O.TERNARY2, O.F16, 64), (O.TERNARY2, O.BF16, 17)])
def test_lockstep_row_tiles_one_kgroup(cuda, fmt, xdt, M):
    # One k-group per workgroup (two workgroups per CU), forced.
    P = O.Problem(fmt, M, 1536, 700, 128, xdt, seed=3800 + M)
    D = DeviceProblem(P)
    with decode_env(LS_KG=1):
        y = D.run()
        assert torch_equal(y, D.run())
    check(y, P.reference(), xdt, f"row tiles one k-group fmt={fmt} M={M}", P)


def test_lockstep_row_tiles_wide_grid(cuda):
    # More 8-tile slabs than CUs (260 on 256 CUs): the planner takes the balanced grid; without
    # it, one k-group per workgroup (two workgroups share a CU) or two rounds of two k-groups.
    N = 16 * 8 * 260
    P = O.Problem(O.INT4, 40, 512, N, 128, O.F16, seed=3900)
    D = DeviceProblem(P)
    y = D.run()
    check(y, P.reference(), O.F16, f"row tiles wide grid N={N}", P)
    with decode_env(LS_BAL=0):
        check(D.run(), P.reference(), O.F16, f"row tiles wide grid, S-piece grid, N={N}", P)
        with decode_env(LS_KG=2):
            check(D.run(), P.reference(), O.F16, f"row tiles wide grid, two k-groups, N={N}", P)


# Balanced grid (several row tiles, more slabs than CUs): every workgroup an equal run of
# (slab, k-block) units, first and last slabs shared with the neighbours through the
# workspace. Slab counts just above the CUs, two and three slabs per workgroup (middle
# slabs whole), K of one to three k-blocks per slab boundary, every format and dtype.
@pytest.mark.parametrize("fmt,xdt,M,K,slabs", [(O.INT4, O.F16, 40, 512, 260), (O.INT4, O.BF16, 80, 1024, 300),
                                                (O.TERNARY2, O.F16, 33, 768, 520), (O.TERNARY2, O.BF16, 64, 384, 770),
                                                (O.INT4, O.F16, 17, 128, 257), (O.INT4, O.F16, 80, 2048, 272)])
def test_lockstep_balanced_grid(cuda, fmt, xdt, M, K, slabs):
    N = 16 * 8 * slabs - 8 * (slabs % 3)  # the last slab's last tile ragged for some
    P = O.Problem(fmt, M, K, N, 128, xdt, seed=4000 + slabs)
    D = DeviceProblem(P)
    with decode_env(LS_BAL=1):
        assert "balanced grid" in hq.describe(fmt, xdt, M, K, N, 128)
        y = D.run()
        assert torch_equal(y, D.run())  # deterministic: partials summed in workgroup order
    check(y, P.reference(), xdt, f"balanced grid fmt={fmt} M={M} K={K} slabs={slabs}", P)


# The same with one row tile (M <= 16), as the planner takes int4 weights of up to 1.25 slabs
# per CU; ternary weights and M = 1 forced.
@pytest.mark.parametrize("fmt,xdt,M,K,slabs", [(O.INT4, O.F16, 12, 512, 260), (O.INT4, O.BF16, 16, 1024, 300),
                                                (O.TERNARY2, O.F16, 9, 768, 270), (O.TERNARY2, O.BF16, 16, 384, 520),
                                                (O.INT4, O.F16, 1, 128, 257)])
def test_lockstep_balanced_grid_one_row_tile(cuda, fmt, xdt, M, K, slabs):
    N = 16 * 8 * slabs - 8 * (slabs % 3)
    P = O.Problem(fmt, M, K, N, 128, xdt, seed=4050 + slabs)
    D = DeviceProblem(P)
    with decode_env(KERNEL=1, LS_BAL=1):
        desc = hq.describe(fmt, xdt, M, K, N, 128)
        assert "MT=1>" in desc and "balanced grid" in desc, desc
        y = D.run()
        assert torch_equal(y, D.run())
    if fmt == O.INT4 and slabs <= 320:
        with decode_env(KERNEL=1):
            assert "balanced grid" in hq.describe(fmt, xdt, M, K, N, 128)  # the planner's own choice
    check(y, P.reference(), xdt, f"balanced grid one row tile fmt={fmt} M={M} K={K} slabs={slabs}", P)


def test_lockstep_balanced_grid_fused_and_counters(cuda):
    # Segment boundaries inside workgroup ranges; the arrival counters return to zero in a
    # caller workspace reused by a second call.
    import torch

    K, M = 640, 48
    Ns = [16 * 8 * 150 + 16, 1000, 16 * 8 * 120]
    probs = [O.Problem(O.INT4, M, K, n, 128, O.F16, seed=4100 + i) for i, n in enumerate(Ns)]
    for p in probs[1:]:
        p.X = probs[0].X
    devs = [DeviceProblem(p) for p in probs]
    segs = [(d.Wp, d.S, d.P.N) for d in devs]
    with decode_env(LS_BAL=1):
        nbytes = hq.workspace_bytes_fused(O.INT4, M, K, [n for n in Ns], 128)
        ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
        outs = hq.gemm_fused(O.INT4, devs[0].X, segs, workspace=ws)
        outs2 = hq.gemm_fused(O.INT4, devs[0].X, segs, workspace=ws)
    for d, y, y2 in zip(devs, outs, outs2):
        check(y, d.P.reference(), O.F16, f"balanced grid fused N={d.P.N}", d.P)
        assert torch_equal(y, y2)
    torch.cuda.synchronize()
    assert int(ws[:65536].view(torch.int32).abs().sum().item()) == 0


def test_lockstep_row_tiles_fused_and_vs_prefill(cuda):
    Ns, K, M = [600, 130, 1000], 1024, 70
    probs = [O.Problem(O.INT4, M, K, n, 128, O.F16, seed=3700 + i) for i, n in enumerate(Ns)]
    for p in probs[1:]:
        p.X = probs[0].X
    devs = [DeviceProblem(p) for p in probs]
    segs = [(d.Wp, d.S, d.P.N) for d in devs]
    outs = hq.gemm_fused(O.INT4, devs[0].X, segs)
    with prefill_env():
        outs_p = hq.gemm_fused(O.INT4, devs[0].X, segs)  # the MFMA tile kernel on the same rows
    for d, y, yp in zip(devs, outs, outs_p):
        check(y, d.P.reference(), O.F16, f"row tiles fused N={d.P.N}", d.P)
        assert O.normwise_error(to_host_f32(y), to_host_f32(yp)) <= OUT_TOL[O.F16]
