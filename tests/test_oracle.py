"""Pins the CPU oracle (oracle/hq_oracle.c) before anything is checked against it.

The reference holds no golden vectors for this path (its tests assert bench-JSON
invariants only, hydrogen/tests/test_h08_marlin_gemm.py:39-101); the one fixed input
is the constant repack fill 0x12345678 (hydrogen/src/model/marlin_gemm.cu:648). So the
oracle is pinned by: library conversions (numpy float16, torch bfloat16), the
semantics of the consumer of the repacked layout (marlin_gemm.cu:192-210), numpy
float64 brute force, closed forms and special cases chosen so that a dropped zero
point, a transposed operand or a wrong group index fails.
"""
import numpy as np
import pytest

import oracle as O

RNG = np.random.default_rng(1234)


# ---------------------------------------------------------------- conversions
def test_f16_to_f32_exhaustive_matches_numpy():
    bits = np.arange(65536, dtype=np.uint16)
    mine = O.to_f32(bits, O.F16)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(mine), nan)
    assert np.array_equal(mine[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne():
    rnd = RNG.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    # dense coverage of the fp16 range, subnormals, ties and overflow boundaries
    special = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 65536.0, 2.0**-24, 2.0**-25, 1.5 * 2.0**-25,
                        2.0**-14, 2.0**-14 * (1 - 2.0**-11), 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, np.inf, -np.inf],
                       dtype=np.float32)
    grid = (np.linspace(-70000, 70000, 200001).astype(np.float32))
    small = (RNG.standard_normal(200000) * 1e-5).astype(np.float32)
    x = np.concatenate([rnd.view(np.float32), special, grid, small])
    x = x[~np.isnan(x)]
    mine = O.from_f32(x, O.F16)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(mine, ref)
    nanbits = O.from_f32(np.array([np.nan], dtype=np.float32), O.F16)
    assert np.isnan(nanbits.view(np.float16)[0])


def test_bf16_conversions_match_torch():
    torch = pytest.importorskip("torch")
    bits = np.arange(65536, dtype=np.uint16)
    mine = O.to_f32(bits, O.BF16)
    ref = torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(mine[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    rnd = RNG.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    rnd = rnd[~np.isnan(rnd)]
    mine = O.from_f32(rnd, O.BF16)
    ref = torch.from_numpy(rnd).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(mine, ref)


# ---------------------------------------------------------------- generator
def test_generator_deterministic_and_distributed():
    a = O.gen_normal(7, 1, 200000)
    b = O.gen_normal(7, 1, 200000)
    c = O.gen_normal(7, 2, 200000)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    x = O.to_f32(a, O.F16).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    s = O.to_f32(O.gen_normal(7, 3, 200000, 0.02, True), O.F16).astype(np.float64)
    assert (s >= 0).all() and abs(s.mean() - 0.02 * np.sqrt(2 / np.pi)) < 2e-4
    w = O.gen_int4(7, 4, 512, 256)
    codes = np.stack([(w >> (4 * i)) & 0xF for i in range(8)]).ravel()
    freq = np.bincount(codes, minlength=16) / codes.size
    assert np.allclose(freq, 1 / 16, atol=0.004)
    t = O.gen_ternary(7, 5, 512, 256)
    tc = np.stack([(t >> (2 * i)) & 3 for i in range(16)]).ravel()
    tf = np.bincount(tc, minlength=4) / tc.size
    assert np.allclose(tf[:3], [0.25, 0.5, 0.25], atol=0.005) and tf[3] == 0


# ---------------------------------------------------------------- helpers (independent numpy restatements)
def dense_codes_int4(K, N):
    return RNG.integers(0, 16, size=(K, N), dtype=np.uint32)


def pack_linear_int4(q):
    """numpy packing of dense codes [K][N] into u32 [K/8][N], nibble i <-> k = 8*kw + i."""
    K, N = q.shape
    q8 = q.reshape(K // 8, 8, N)
    return np.bitwise_or.reduce(q8 << (4 * np.arange(8, dtype=np.uint32))[None, :, None], axis=1).astype(np.uint32)


def pack_linear_tern(c):
    K, N = c.shape
    c16 = c.reshape(K // 16, 16, N).astype(np.uint32)
    return np.bitwise_or.reduce(c16 << (2 * np.arange(16, dtype=np.uint32))[None, :, None], axis=1).astype(np.uint32)


# ---------------------------------------------------------------- repack (marlin_gemm.cu:446-455)
def test_repack_ref_constant_fill_known_answer():
    # benchmark_repacking (marlin_gemm.cu:646-657) repacks a constant 0x12345678 fill.
    K, N = 4096, 64
    src = np.full((K // 8) * N, 0x12345678, dtype=np.uint32)
    assert np.array_equal(O.repack_ref(src, K, N), src)


@pytest.mark.parametrize("K,N", [(32, 1), (64, 5), (128, 48), (256, 33)])
def test_repack_ref_matches_consumer_semantics(K, N):
    # kernel_marlin_gemm_int4 reads uint4 quad (kq, n) and takes nibble i of word w_idx
    # as k = 32*kq + 8*w_idx + i of column n (marlin_gemm.cu:192-210).
    q = dense_codes_int4(K, N)
    dst = O.repack_ref(pack_linear_int4(q).ravel(), K, N).reshape(K // 32, N, 4)
    nib = np.stack([(dst >> (4 * i)) & 0xF for i in range(8)], axis=-1)  # [kq, n, w, i]
    recon = nib.transpose(0, 2, 3, 1).reshape(K, N)
    assert np.array_equal(recon, q)


def test_repack_ref_is_a_permutation():
    src = O.gen_int4(3, 9, 256, 40)
    dst = O.repack_ref(src, 256, 40)
    assert np.array_equal(np.sort(src), np.sort(dst))


# ---------------------------------------------------------------- dequant (marlin_gemm.cu:495-512)
def test_dequant_int4_reference_form_and_zero_point():
    K, N, g = 256, 24, 128
    q = dense_codes_int4(K, N)
    q[:16, :16] = np.arange(16, dtype=np.uint32)[:, None]  # every code appears
    s_bits = O.gen_normal(11, 1, (K // g) * N, 0.02, True).reshape(K // g, N)
    s = O.to_f32(s_bits, O.F16)
    wdq = O.dequant(O.INT4, pack_linear_int4(q).ravel(), s_bits.ravel(), K, N, g)
    sk = np.repeat(s, g, axis=0)
    # the reference's exact form, evaluated by numpy in float32 with separate roundings
    ref_form = q.astype(np.float32) * sk + np.float32(-8.0) * sk
    assert np.array_equal(wdq.view(np.uint32), ref_form.view(np.uint32))
    # and within one ulp of the zero-point form (q - 8) * s
    exact = (q.astype(np.float64) - 8.0) * sk.astype(np.float64)
    ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(wdq - exact) <= ulp)
    assert np.all(wdq[q == 8] == 0.0)


def test_dequant_ternary_values():
    K, N, g = 256, 16, 128
    c = RNG.choice([0, 1, 2], size=(K, N)).astype(np.uint32)
    s_bits = O.gen_normal(12, 1, (K // g) * N, 0.02, True).reshape(K // g, N)
    s = O.to_f32(s_bits, O.F16)
    wdq = O.dequant(O.TERNARY2, pack_linear_tern(c).ravel(), s_bits.ravel(), K, N, g)
    expect = (c.astype(np.float32) - 1.0) * np.repeat(s, g, axis=0)
    assert np.array_equal(wdq, expect)
    bad = c.copy()
    bad[5, 3] = 3
    with pytest.raises(ValueError):
        O.dequant(O.TERNARY2, pack_linear_tern(bad).ravel(), s_bits.ravel(), K, N, g)


def test_ternary_nonfinite_scale_drops_group():
    # native_decoder.cu:174: a NaN/Inf block scale skips the block.
    K, N, g = 256, 16, 128
    c = np.full((K, N), 2, dtype=np.uint32)
    s_bits = O.gen_normal(13, 1, (K // g) * N, 0.02, True).reshape(K // g, N)
    s_bits[0, 3] = 0x7E00  # NaN
    s_bits[1, 4] = 0x7C00  # +Inf
    wdq = O.dequant(O.TERNARY2, pack_linear_tern(c).ravel(), s_bits.ravel(), K, N, g)
    assert np.all(wdq[:128, 3] == 0) and np.all(wdq[128:, 4] == 0)
    assert np.all(wdq[128:, 3] > 0)


# ---------------------------------------------------------------- matmul (marlin_gemm.cu:52-70)
def fp32_bound(X, W):
    """|sum_k x w - fl(sum)| <= K * 2^-23 * sum_k |x w| (loose sequential-sum bound)."""
    K = X.shape[1]
    return K * 2.0**-23 * (np.abs(X).astype(np.float64) @ np.abs(W).astype(np.float64)) + 1e-30


@pytest.mark.parametrize("M,K,N", [(1, 37, 5), (3, 64, 17), (7, 300, 41)])
def test_gemm_f32_against_float64(M, K, N):
    X = RNG.standard_normal((M, K)).astype(np.float32)
    W = RNG.standard_normal((K, N)).astype(np.float32)
    Y = O.gemm_f32(X, W)
    ref = X.astype(np.float64) @ W.astype(np.float64)
    assert np.all(np.abs(Y - ref) <= fp32_bound(X, W))


def test_gemm_f32_first_term_and_orientation():
    # Y = X W with X [M,K] and W [K,N]: a transposed operand cannot pass on a 2x3x4 case.
    X = np.arange(6, dtype=np.float32).reshape(2, 3)
    W = np.arange(12, dtype=np.float32).reshape(3, 4)
    assert np.array_equal(O.gemm_f32(X, W), (X @ W).astype(np.float32))


def make_problem_arrays(fmt, M, K, N, g, xdtype, seed):
    P = O.Problem(fmt, M, K, N, g, xdtype, seed)
    return P


@pytest.mark.parametrize("fmt", [O.INT4, O.TERNARY2])
@pytest.mark.parametrize("xdtype", [O.F16, O.BF16])
def test_qgemm_equals_dequant_then_gemm_bitwise(fmt, xdtype):
    P = O.Problem(fmt, 5, 384, 40, 128, xdtype, seed=21)
    Y = P.reference()
    Wdq = O.dequant(fmt, P.W, P.scales.ravel(), P.K, P.N, P.group)
    Y2 = O.gemm_f32(O.to_f32(P.X, xdtype), Wdq)
    assert np.array_equal(Y.view(np.uint32), Y2.view(np.uint32))


@pytest.mark.parametrize("fmt", [O.INT4, O.TERNARY2])
def test_qgemm_against_float64(fmt):
    P = O.Problem(fmt, 4, 512, 48, 128, O.F16, seed=22)
    Y = P.reference()
    X = O.to_f32(P.X, O.F16)
    Wdq = O.dequant(fmt, P.W, P.scales.ravel(), P.K, P.N, P.group)
    ref = X.astype(np.float64) @ Wdq.astype(np.float64)
    assert np.all(np.abs(Y - ref) <= fp32_bound(X, Wdq))


def test_qgemm_thread_count_invariant():
    P = O.Problem(O.INT4, 6, 1024, 300, 128, O.F16, seed=23)
    a = P.reference(threads=1)
    b = P.reference(threads=8)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_qgemm_zero_point_code_gives_zero():
    K, N, M = 256, 32, 3
    W = np.full((K // 8) * N, 0x88888888, dtype=np.uint32)
    X = O.gen_normal(1, 1, M * K).reshape(M, K)
    S = O.gen_normal(1, 2, (K // 128) * N, 0.02, True)
    assert np.all(O.qgemm(O.INT4, X, O.F16, W, S, N) == 0.0)
    T = np.full((K // 16) * N, 0x55555555, dtype=np.uint32)  # all c = 1, t = 0
    assert np.all(O.qgemm(O.TERNARY2, X, O.F16, T, S, N) == 0.0)


@pytest.mark.parametrize("fmt", [O.INT4, O.TERNARY2])
def test_qgemm_one_hot_rows_select_weight_rows(fmt):
    K, N, g = 384, 24, 128
    P = O.Problem(fmt, 1, K, N, g, O.F16, seed=24)
    ks = [0, 1, 127, 128, 200, 383]
    X = np.zeros((len(ks), K), dtype=np.uint16)
    for r, k in enumerate(ks):
        X[r, k] = 0x3C00  # 1.0
    Y = O.qgemm(fmt, X, O.F16, P.W, P.scales.ravel(), N, g)
    Wdq = O.dequant(fmt, P.W, P.scales.ravel(), K, N, g)
    assert np.array_equal(Y, Wdq[ks])


# ---------------------------------------------------------------- caller bias, small groups
# The reference's forward takes any per-group fp32 bias (marlin_gemm.hpp:100-107) and reads
# one scale and bias per 32-wide chunk (marlin_gemm.cu:191-196), so groups of 32 and 64 are valid.
@pytest.mark.parametrize("g", [32, 64, 128, 256])
def test_dequant_int4_bias_reference_form(g):
    K, N = 512, 24
    q = dense_codes_int4(K, N)
    s_bits = O.gen_normal(12, 1, (K // g) * N, 0.02, True).reshape(K // g, N)
    b = (RNG.standard_normal((K // g, N)) * 0.05).astype(np.float32)
    wdq = O.dequant_int4_bias(pack_linear_int4(q).ravel(), s_bits, b, K, N, g)
    sk = np.repeat(O.to_f32(s_bits, O.F16), g, axis=0)
    bk = np.repeat(b, g, axis=0)
    # numpy float32: q * s rounded, then + b rounded (the reference's host form)
    ref = q.astype(np.float32) * sk + bk
    assert np.array_equal(wdq.view(np.uint32), ref.view(np.uint32))
    # a group index off by one (k // g + 1) or a transposed bias would not match
    assert not np.array_equal(wdq, q.astype(np.float32) * sk + np.roll(bk, g, axis=0))


@pytest.mark.parametrize("g", [32, 128])
def test_bias_minus_8s_is_the_zero_point_form_bitwise(g):
    P = O.Problem(O.INT4, 5, 512, 40, g, O.F16, seed=23, bias="minus8s")
    Yb = P.reference()
    Y0 = O.qgemm(O.INT4, P.X, O.F16, P.W, P.scales, P.N, g)
    assert np.array_equal(Yb.view(np.uint32), Y0.view(np.uint32))
    Wb = O.dequant_int4_bias(P.W, P.scales, P.bias, P.K, P.N, g)
    W0 = O.dequant(O.INT4, P.W, P.scales.ravel(), P.K, P.N, g)
    assert np.array_equal(Wb.view(np.uint32), W0.view(np.uint32))
    # NULL bias is the same function
    Yn = O.qgemm_bias(P.X, O.F16, P.W, P.scales, None, P.N, g)
    assert np.array_equal(Yn.view(np.uint32), Y0.view(np.uint32))


@pytest.mark.parametrize("g", [32, 64, 128])
def test_qgemm_bias_against_float64(g):
    P = O.Problem(O.INT4, 4, 512, 48, g, O.F16, seed=24, bias="random")
    Y = P.reference()
    X = O.to_f32(P.X, O.F16)
    Wdq = O.dequant_int4_bias(P.W, P.scales, P.bias, P.K, P.N, g)
    ref = X.astype(np.float64) @ Wdq.astype(np.float64)
    assert np.all(np.abs(Y - ref) <= fp32_bound(X, Wdq))
    # equals dequant-then-gemm bit for bit
    assert np.array_equal(Y.view(np.uint32), O.gemm_f32(X, Wdq).view(np.uint32))


def test_qgemm_bias_constant_code_closed_form():
    # constant code c: Y[m, n] = sum_g (c s[g, n] + b[g, n]) * sum_{k in g} x[m, k], groups of 32
    K, N, g, M, c = 512, 20, 32, 3, 5
    W = np.full((K // 8) * N, int("".join([f"{c:x}"] * 8), 16), dtype=np.uint32)
    X = O.gen_normal(3, 1, M * K).reshape(M, K)
    S = O.gen_normal(3, 2, (K // g) * N, 0.02, True).reshape(K // g, N)
    B = (RNG.standard_normal((K // g, N)) * 0.05).astype(np.float32)
    Y = O.qgemm_bias(X, O.F16, W, S, B, N, g)
    xf = O.to_f32(X, O.F16).astype(np.float64)
    wg = c * O.to_f32(S, O.F16).astype(np.float64) + B.astype(np.float64)  # [G, N]
    ref = xf.reshape(M, K // g, g).sum(axis=2) @ wg
    assert np.allclose(Y, ref, rtol=1e-5, atol=1e-5)


def test_qgemm_constant_code_closed_form():
    # constant code c: Y[m, n] = sum_g (c - 8) * s[g, n] * sum_{k in g} x[m, k]
    K, N, g, M, c = 512, 20, 128, 3, 13
    W = np.full((K // 8) * N, int("".join([f"{c:x}"] * 8), 16), dtype=np.uint32)
    X = O.gen_normal(2, 1, M * K).reshape(M, K)
    S = O.gen_normal(2, 2, (K // g) * N, 0.02, True).reshape(K // g, N)
    Y = O.qgemm(O.INT4, X, O.F16, W, S.ravel(), N, g)
    xf = O.to_f32(X, O.F16).astype(np.float64)
    sf = O.to_f32(S, O.F16).astype(np.float64)
    gsum = xf.reshape(M, K // g, g).sum(axis=2)  # [M, G]
    ref = (c - 8) * gsum @ sf
    assert np.allclose(Y, ref, rtol=1e-5, atol=1e-6)


def test_fidelity_matches_numpy():
    a = RNG.standard_normal(1000).astype(np.float32)
    b = a + RNG.standard_normal(1000).astype(np.float32) * 1e-3
    mx, mse = O.fidelity(a, b)
    d = np.abs(a.astype(np.float64) - b.astype(np.float64))
    assert mx == d.max() and np.isclose(mse, (d * d).mean())


def test_golden_fixture_pins_oracle():
    from pathlib import Path

    path = Path(__file__).resolve().parent / "golden" / "qgemm_small.npz"
    data = np.load(path)
    for case in sorted({k.split("/")[0] for k in data.files}):
        fmt = int(data[f"{case}/fmt"])
        xdt = int(data[f"{case}/xdtype"])
        X, W, S = data[f"{case}/X"], data[f"{case}/W"], data[f"{case}/scales"]
        expect = data[f"{case}/Y64"]
        N = int(data[f"{case}/N"])
        Y = O.qgemm(fmt, X, xdt, W, S.ravel(), N, int(data[f"{case}/group"]))
        Xf = O.to_f32(X, xdt)
        Wdq = O.dequant(fmt, W, S.ravel(), X.shape[1], N, int(data[f"{case}/group"]))
        assert np.all(np.abs(Y - expect) <= fp32_bound(Xf, Wdq)), case


# ---------------------------------------------------------------- GGUF TQ1_0 (native_decoder.cu:31-36, 87-101)
def tq1_block(trit_bytes, d_bits=0x3C00):
    b = np.zeros(O.TQ1_0_BLOCK_BYTES, dtype=np.uint8)
    b[0], b[1] = d_bits & 0xFF, d_bits >> 8
    b[2:54] = trit_bytes
    return b


def test_tq1_0_constant_bytes():
    # 0 -> every digit 0 (t = -1); 121 = 11111 in base 3 (t = 0); 242 = 22222 (t = +1).
    for byte, c in ((0, 0), (121, 1), (242, 2)):
        assert np.all(O.tq1_0_codes(tq1_block(byte)) == c)
    assert O.tq1_0_scale(tq1_block(0, 0xBEEF)) == 0xBEEF


def test_tq1_0_encode_decode_round_trip():
    # Encode chosen trits the way a writer would (Horner, least significant digit first:
    # element 5j + s is digit s of byte j; elements 250 + 3j + s digit s of byte 50 + j),
    # then decode with the oracle. A wrong digit order, byte index or offset fails.
    rng = np.random.default_rng(7)
    for _ in range(20):
        codes = rng.integers(0, 3, 256)
        trit_bytes = np.zeros(52, dtype=np.int64)
        for j in range(50):
            trit_bytes[j] = sum(int(codes[5 * j + s]) * 3**s for s in range(5))
        for j in range(2):
            trit_bytes[50 + j] = sum(int(codes[250 + 3 * j + s]) * 3**s for s in range(3))
        assert trit_bytes.max() <= 242
        assert np.array_equal(O.tq1_0_codes(tq1_block(trit_bytes.astype(np.uint8))), codes)


def test_tq1_0_bytes_above_242_decode_digit_by_digit():
    # 255 = 100110 in base 3: digits (least first) 0, 1, 1, 0, 0 (the sixth is dropped); 243 = 100000.
    c = O.tq1_0_codes(tq1_block(np.array([255] * 50 + [255, 243], dtype=np.uint8)))
    assert list(c[:5]) == [0, 1, 1, 0, 0]
    assert list(c[250:253]) == [0, 1, 1] and list(c[253:256]) == [0, 0, 0]


def test_tq1_0_gemv_closed_forms():
    K, N = 512, 3
    blocks = np.stack([np.stack([tq1_block(242, 0x3800), tq1_block(0, 0x4000)]),     # +0.5 then -2.0
                       np.stack([tq1_block(121, 0x3C00), tq1_block(242, 0x7C00)]),   # zeros, Inf d (skipped)
                       np.stack([tq1_block(0, 0x7E00), tq1_block(121, 0x3C00)])])    # NaN d (skipped), zeros
    X = np.random.default_rng(3).standard_normal((2, K)).astype(np.float32)
    Y = O.gemv_tq1_0(X, blocks, N)
    ref0 = 0.5 * X[:, :256].astype(np.float64).sum(1) - 2.0 * X[:, 256:].astype(np.float64).sum(1)
    np.testing.assert_allclose(Y[:, 0], ref0, rtol=1e-5, atol=1e-4)
    assert np.all(Y[:, 1] == 0) and np.all(Y[:, 2] == 0)


def test_tq1_0_gemv_matches_float64_brute_force():
    K, N, M = 768, 5, 3
    blocks = O.gen_tq1_0(5, N, K)
    X = np.random.default_rng(4).standard_normal((M, K)).astype(np.float32)
    W = np.zeros((K, N))
    for n in range(N):
        for b in range(K // 256):
            d = np.uint16(O.tq1_0_scale(blocks[n, b])).view(np.float16).astype(np.float64)
            W[256 * b:256 * (b + 1), n] = d * (O.tq1_0_codes(blocks[n, b]).astype(np.float64) - 1)
    np.testing.assert_allclose(O.gemv_tq1_0(X, blocks, N), X.astype(np.float64) @ W, rtol=1e-4, atol=1e-4)


# ---------------------------------------------------------------- the int8 path
# kernel_cutlass_int8_gemm (hydrogen/src/model/marlin_gemm.cu:327-377): activations quantised as
# static_cast<int8_t>(fminf(fmaxf(x * 127, -128), 127)) (:356-359), weights q * 16 - 128 (:508),
# per-quad integer dot products accumulated as fp32 dot * (1 / 127), times scales[col] (:371-375).
def test_quantize_x_int8_known_answers():
    # Conversion toward zero (not rounding: 0.5 -> 63, not 64), clamping at both ends, and NaN
    # to -128 (fmaxf returns the non-NaN operand, then fminf keeps -128).
    cases = {1.0: 127, -1.0: -127, 0.5: 63, -0.5: -63, 1e-3: 0, -1e-3: 0, 2.0: 127, -2.0: -128, -1.01: -128,
             1.007: 127, 0.99999: 126, float("inf"): 127, float("-inf"): -128, float("nan"): -128}
    for x, q in cases.items():
        assert O.quantize_x_int8(x) == q, (x, O.quantize_x_int8(x), q)


def test_int8_from_int4_is_16q_minus_128():
    K, N = 256, 12
    q = dense_codes_int4(K, N)
    w8 = O.int8_from_int4(pack_linear_int4(q).ravel(), K, N)
    assert np.array_equal(w8.astype(np.int32), q.astype(np.int32) * 16 - 128)
    assert w8.min() == -128 and w8.max() == 112


def int8_problem(M, K, N, seed):
    rng = np.random.default_rng(seed)
    X = (rng.standard_normal((M, K)) * 0.4).astype(np.float32)
    W = (rng.integers(0, 16, (K, N)) * 16 - 128).astype(np.int8)
    s = (np.abs(rng.standard_normal(N)) * 0.02 + 1e-3).astype(np.float32)
    return X, W, s


@pytest.mark.parametrize("M,K,N", [(1, 128, 40), (5, 512, 33), (8, 4096, 64), (16, 1024, 17)])
def test_gemm_int8_against_integer_float64(M, K, N):
    X, W, s = int8_problem(M, K, N, M + K + N)
    Y = O.gemm_int8(X, W, s)
    xq = np.array([[O.quantize_x_int8(v) for v in row] for row in X], dtype=np.int64)
    dots = xq.reshape(M, K // 4, 4, 1) * W.astype(np.int64).reshape(1, K // 4, 4, N)
    quad = dots.sum(axis=2)                       # [M, K/4, N] exact integers
    exact = quad.sum(axis=1) / 127.0 * s.astype(np.float64)
    # fp32 accumulation of K / 4 terms (one rounding each) and the final product
    bound = (K // 4 + 2) * 2.0**-24 * (np.abs(quad).sum(axis=1) / 127.0) * np.abs(s) + 1e-30
    assert np.all(np.abs(Y - exact) <= bound)
    # A rounding (not truncating) quantiser, or a scale row other than the first, fails this.
    xr = np.clip(np.rint(X * 127), -128, 127).astype(np.int64)
    alt = (xr @ W.astype(np.int64)) / 127.0 * s
    assert not np.all(np.abs(Y - alt) <= bound)


def test_gemm_int8_known_answers():
    # x = 1 -> 127; every weight 16 (code 9): each quad contributes fp32(4 * 127 * 16 / 127).
    K, N = 256, 3
    X = np.ones((2, K), dtype=np.float32)
    X[1, :] = 0.0
    X[1, 7] = -1.0
    W = np.full((K, N), 16, dtype=np.int8)
    s = np.array([1.0, 0.5, 2.0], dtype=np.float32)
    Y = O.gemm_int8(X, W, s)
    # fmaf(dot, 1/127, acc) emulated exactly: the product of an integer below 2^13 and a 24-bit
    # significand is exact in float64, and so is its sum with the fp32 accumulator.
    acc = np.float32(0.0)
    for _ in range(K // 4):
        acc = np.float32(np.float64(acc) + np.float64(4 * 127 * 16) * np.float64(np.float32(1.0 / 127.0)))
    assert np.array_equal(Y[0], acc * s)
    # one nonzero activation: the single quad holding k = 7 gives -127 * 16 / 127 = -16 exactly
    assert np.allclose(Y[1], np.float32(-127 * 16) * np.float32(1.0 / 127.0) * s, rtol=1e-7)
    # thread count does not change the bits
    X2, W2, s2 = int8_problem(3, 512, 50, 7)
    assert np.array_equal(O.gemm_int8(X2, W2, s2, threads=1).view(np.uint32),
                          O.gemm_int8(X2, W2, s2, threads=8).view(np.uint32))
