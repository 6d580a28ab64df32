"""CPU tests of the C ABI: the library loads, exports what include/hq_qgemm.h declares,
rejects bad arguments before touching a device, and its host repacks are bijections
whose reference layout is bit-exact with the oracle's restatement of
hydrogen/src/model/marlin_gemm.cu:446-455."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from nebula_amd import hq

ROOT = Path(__file__).resolve().parent.parent


def header_functions():
    text = (ROOT / "include" / "hq_qgemm.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = hq.lib()
    declared = header_functions()
    assert declared == sorted(hq.EXPORTS)
    for name in declared:
        assert hasattr(L, name), name
    assert "gfx950" in hq.version()


def test_status_strings():
    L = hq.lib()
    assert L.hq_status_string(0) == b"ok"
    assert L.hq_status_string(6) == b"invalid ternary code"


def test_sizes():
    assert hq.linear_words(hq.FORMAT_INT4, 4096, 4096) == 512 * 4096
    assert hq.linear_words(hq.FORMAT_TERNARY2, 5120, 27648) == 320 * 27648
    assert hq.packed_words(hq.FORMAT_INT4, 4096, 4096) == 4096 * 4096 // 8
    assert hq.packed_words(hq.FORMAT_INT4, 128, 17) == 2 * 256  # N padded to 32
    assert hq.packed_words(hq.FORMAT_TERNARY2, 256, 16) == 2 * 128
    assert hq.packed_words(hq.FORMAT_INT4, 100, 16) == 0


def workspace_bytes(fmt, M, K, N, group=128):
    b = ctypes.c_size_t(99)
    st = hq.lib().hq_workspace_bytes(fmt, M, K, N, group, ctypes.byref(b))
    return st, b.value


def workspace_bytes_fused(fmt, M, K, Ns, group=128, bias=0):
    arr = (ctypes.c_uint32 * len(Ns))(*Ns)
    b = ctypes.c_size_t(99)
    st = hq.lib().hq_workspace_bytes_fused(fmt, M, K, group, arr, len(Ns), bias, ctypes.byref(b))
    return st, b.value


def test_workspace_bytes():
    # Large decode shapes with few column tiles whose activation rows do not fit in LDS
    # cut their slabs along K and need a fix-up workspace: a fixed counter area plus fp32
    # partial tiles that scale with M. With the rows in LDS (M <= 2 at K = 27648) the
    # X-resident kernel needs none.
    st, b16 = workspace_bytes_fused(hq.FORMAT_INT4, 16, 27648, [5120])
    st4, b4 = workspace_bytes_fused(hq.FORMAT_INT4, 4, 27648, [5120])
    assert st == st4 == hq.HQ_OK
    assert b16 > b4 > 0 and b16 % 256 == 0 and b4 % 256 == 0
    assert workspace_bytes_fused(hq.FORMAT_INT4, 1, 27648, [5120]) == (hq.HQ_OK, 0)
    # hq_workspace_bytes covers the call with and without a bias.
    for M in (1, 16):
        plain = workspace_bytes_fused(hq.FORMAT_INT4, M, 27648, [5120])[1]
        biased = workspace_bytes_fused(hq.FORMAT_INT4, M, 27648, [5120], bias=1)[1]
        assert workspace_bytes(hq.FORMAT_INT4, M, 27648, 5120) == (hq.HQ_OK, max(plain, biased))
    # Up to M = 80 the streaming kernel runs (row tiles of 16): its partials grow with the
    # row tiles.
    _, d16 = workspace_bytes(hq.FORMAT_INT4, 16, 4096, 4096)
    _, d80 = workspace_bytes(hq.FORMAT_INT4, 80, 4096, 4096)
    assert d16 > 65536 and d80 - 65536 == 5 * (d16 - 65536)
    # Prefill shapes (M > 80) too get exactly what the call asks for (with or without a bias):
    # grids of whole tiles need none, stream-K grids the counter area plus two fp32 partial
    # tiles per stream-K workgroup; K < 1024 is never split along K.
    for fmt, M, K, N in [(hq.FORMAT_INT4, 81, 4096, 4096), (hq.FORMAT_INT4, 300, 5120, 16),
                         (hq.FORMAT_TERNARY2, 2048, 5120, 27648), (hq.FORMAT_TERNARY2, 2048, 5120, 16),
                         (hq.FORMAT_INT4, 1024, 5120, 7168), (hq.FORMAT_INT4, 2048, 896, 4096)]:
        exact = workspace_bytes_fused(fmt, M, K, [N])[1]
        if fmt == hq.FORMAT_INT4:
            exact = max(exact, workspace_bytes_fused(fmt, M, K, [N], bias=1)[1])
        assert workspace_bytes(fmt, M, K, N) == (hq.HQ_OK, exact), (fmt, M, K, N)
    assert workspace_bytes(hq.FORMAT_TERNARY2, 2048, 5120, 27648) == (hq.HQ_OK, 0)  # 1728 whole tiles
    _, p16 = workspace_bytes(hq.FORMAT_TERNARY2, 2048, 5120, 16)  # 32 tiles on 256 stream-K workgroups
    assert p16 > 65536 and (p16 - 65536) % (2 * 64 * 256 * 4) == 0
    assert workspace_bytes(hq.FORMAT_INT4, 2048, 896, 4096) == (hq.HQ_OK, 0)
    # Groups that are multiples of 32 are sized (the general kernels), bad shapes reported.
    assert workspace_bytes(hq.FORMAT_INT4, 16, 4096, 4096, group=64)[0] == hq.HQ_OK
    assert workspace_bytes(hq.FORMAT_INT4, 16, 4000, 4096)[0] == hq.HQ_ERR_SHAPE
    assert workspace_bytes(hq.FORMAT_INT4, 16, 4096, 4096, group=48)[0] == hq.HQ_ERR_SHAPE
    assert workspace_bytes(hq.FORMAT_INT4, 16, 4096, 4096, group=96)[0] == hq.HQ_ERR_SHAPE  # K % group
    assert workspace_bytes(hq.FORMAT_INT4, 0, 4096, 4096)[0] == hq.HQ_ERR_SHAPE
    assert workspace_bytes(7, 16, 4096, 4096)[0] == hq.HQ_ERR_INVALID_ARG


def test_workspace_bytes_fused_is_what_the_call_asks_for():
    # A fused call needs exactly hq_workspace_bytes_fused bytes: one byte less is rejected
    # with HQ_ERR_WORKSPACE before any launch, the exact size passes validation (and would
    # launch, so the check stops at the size by giving it a misaligned buffer).
    L = hq.lib()
    cases = [(hq.FORMAT_INT4, 8, 1024, [16] * 8), (hq.FORMAT_INT4, 3, 27648, [5120, 1024]),
             (hq.FORMAT_TERNARY2, 16, 5120, [5120, 1024, 1024]), (hq.FORMAT_INT4, 80, 4096, [600, 130, 1000]),
             (hq.FORMAT_INT4, 40, 2048, [16, 32, 48, 64]), (hq.FORMAT_TERNARY2, 1, 17408, [5120])]
    for fmt, M, K, Ns in cases:
        st, need = workspace_bytes_fused(fmt, M, K, Ns)
        assert st == hq.HQ_OK
        if need == 0:
            continue
        segs = (hq.Segment * len(Ns))()
        for i, n in enumerate(Ns):
            segs[i] = hq.Segment(0x2000, 0x3000, None, 0x4000, n, n)
        assert L.hq_gemm_fused(0x1000, 1, K, fmt, segs, len(Ns), M, K, 128, 0x10000, need - 1, None) == \
            hq.HQ_ERR_WORKSPACE, (fmt, M, K, Ns)
        assert L.hq_gemm_fused(0x1000, 1, K, fmt, segs, len(Ns), M, K, 128, 0x10010, need, None) == \
            hq.HQ_ERR_ALIGNMENT, (fmt, M, K, Ns)
    # The case the single-shape rule under-sized: eight 16-column int4 segments at M = 8
    # (with a bias: the lockstep kernel, which cuts slabs along K).
    need8 = workspace_bytes_fused(hq.FORMAT_INT4, 8, 1024, [16] * 8, bias=1)[1]
    assert need8 >= workspace_bytes_fused(hq.FORMAT_INT4, 8, 1024, [16 * 8], bias=1)[1] > 0
    assert workspace_bytes_fused(hq.FORMAT_INT4, 8, 1024, [])[0] == hq.HQ_ERR_INVALID_ARG
    assert workspace_bytes_fused(hq.FORMAT_INT4, 8, 1024, [0])[0] == hq.HQ_ERR_SHAPE
    assert workspace_bytes_fused(hq.FORMAT_TERNARY2, 8, 1024, [64], bias=1)[0] == hq.HQ_ERR_UNSUPPORTED


def test_describe_gemm_names_the_kernel_families(monkeypatch):
    assert hq.describe(hq.FORMAT_INT4, hq.DTYPE_F16, 1, 27648, 5120).startswith("hq_decode_xr_kernel<int4,f16,")
    assert "x 3 pieces" in hq.describe(hq.FORMAT_INT4, hq.DTYPE_F16, 4, 27648, 5120)
    assert "x 3 pieces" in hq.describe(hq.FORMAT_INT4, hq.DTYPE_F16, 8, 27648, 5120)
    with monkeypatch.context() as m:
        m.setenv("HQ_DECODE_KERNEL", "0")
        assert hq.describe(hq.FORMAT_INT4, hq.DTYPE_F16, 4, 27648, 5120).startswith("hq_decode_kernel<int4,f16,")
    assert hq.describe(hq.FORMAT_INT4, hq.DTYPE_F16, 16, 5120, 27648).startswith(
        "hq_decode_xr_kernel<int4,f16,T=4,U=2,SG=2>")
    assert hq.describe(hq.FORMAT_INT4, hq.DTYPE_F16, 16, 5120, 69632).startswith("hq_decode_ls_kernel<int4,f16,")
    assert hq.describe(hq.FORMAT_INT4, hq.DTYPE_F16, 20, 5120, 27648).startswith("hq_decode_ls_kernel<int4,f16,")
    assert hq.describe(hq.FORMAT_TERNARY2, hq.DTYPE_BF16, 2048, 5120, 27648).startswith(
        "hq_prefill_kernel<ternary2,bf16")
    assert "general" in hq.describe(hq.FORMAT_INT4, hq.DTYPE_F16, 4, 4096, 4096, group=32)
    assert "general" in hq.describe(hq.FORMAT_INT4, hq.DTYPE_BF16, 300, 4096, 4096, with_bias=True)
    with pytest.raises(hq.HQError):
        hq.describe(hq.FORMAT_TERNARY2, hq.DTYPE_F16, 4, 4096, 4096, with_bias=True)


def test_device_status_without_faults():
    # No kernel has run: the fault word was never set (nor allocated).
    assert hq.lib().hq_last_error() is not None


def test_workspace_checked_before_launch():
    L = hq.lib()
    _, need = workspace_bytes(hq.FORMAT_INT4, 16, 27648, 5120)
    need = workspace_bytes_fused(hq.FORMAT_INT4, 16, 27648, [5120])[1]
    args = (0x1000, 1, 27648, 0x2000, 0x3000, None, 0x4000, 5120, 16, 27648, 5120, 128)
    assert L.hq_gemm_w4a16(*args, 0x10000, need - 1, None) == hq.HQ_ERR_WORKSPACE
    assert b"smaller" in L.hq_last_error()
    assert L.hq_gemm_w4a16(*args, 0x10010, need, None) == hq.HQ_ERR_ALIGNMENT


# ---------------------------------------------------------------- validation (no device work)
def call_gemm(X=0x1000, dtype=1, ldx=4096, Wp=0x2000, S=0x3000, Y=0x4000, ldy=4096, M=16, K=4096, N=4096, g=128,
              fn="hq_gemm_w4a16", bias=None):
    if fn == "hq_gemm_w4a16":
        return hq.lib().hq_gemm_w4a16(X, dtype, ldx, Wp, S, bias, Y, ldy, M, K, N, g, None, 0, None)
    return getattr(hq.lib(), fn)(X, dtype, ldx, Wp, S, Y, ldy, M, K, N, g, None, 0, None)


@pytest.mark.parametrize("kw,status", [
    (dict(X=0), hq.HQ_ERR_INVALID_ARG),
    (dict(Wp=0), hq.HQ_ERR_INVALID_ARG),
    (dict(S=0), hq.HQ_ERR_INVALID_ARG),
    (dict(Y=0), hq.HQ_ERR_INVALID_ARG),
    (dict(dtype=3), hq.HQ_ERR_INVALID_ARG),
    (dict(M=0), hq.HQ_ERR_SHAPE),
    (dict(N=0), hq.HQ_ERR_SHAPE),
    (dict(K=4000, ldx=4000), hq.HQ_ERR_SHAPE),
    (dict(g=48), hq.HQ_ERR_SHAPE),
    (dict(g=96), hq.HQ_ERR_SHAPE),
    (dict(K=384, ldx=384, g=256), hq.HQ_ERR_SHAPE),
    (dict(ldx=4000), hq.HQ_ERR_SHAPE),
    (dict(ldy=100), hq.HQ_ERR_SHAPE),
    (dict(ldx=4100), hq.HQ_ERR_ALIGNMENT),
    (dict(X=0x1008), hq.HQ_ERR_ALIGNMENT),
    (dict(Wp=0x2004), hq.HQ_ERR_ALIGNMENT),
    (dict(S=0x3001), hq.HQ_ERR_ALIGNMENT),
    (dict(Y=0x4001), hq.HQ_ERR_ALIGNMENT),
])
def test_gemm_rejects_bad_arguments(kw, status):
    for fn in ("hq_gemm_w4a16", "hq_gemm_w2a16"):
        assert call_gemm(fn=fn, **kw) == status
        assert hq.lib().hq_last_error().decode()


# Operands of 2 GiB or more: the kernels address every operand with 32-bit byte offsets, so
# the entry points reject such shapes (HQ_ERR_SHAPE, no device work) instead of reading zeros
# past the wrapped range.
@pytest.mark.parametrize("kw,what", [
    (dict(M=16, ldx=1 << 26), "X spans"),                                  # 16 * 2^26 * 2 = 2 GiB
    (dict(M=16, ldy=1 << 26), "Y spans"),
    (dict(M=1, K=4096, N=1 << 26, ldy=1 << 26), "scales"),                 # 32 rows * 2^26 * 2 B
    (dict(M=1, K=1 << 16, ldx=1 << 16, N=1 << 16, ldy=1 << 16), "packed weights"),  # 2^12 tiles * 512 * 1 KiB
])
def test_gemm_rejects_operands_beyond_32_bit_offsets(kw, what):
    assert call_gemm(**kw) == hq.HQ_ERR_SHAPE
    assert what in hq.lib().hq_last_error().decode()
    # One below each limit passes validation (and fails later only for the fake pointers).
    if what == "X spans":
        assert call_gemm(M=16, ldx=(1 << 26) - 8) != hq.HQ_ERR_SHAPE
    if what == "packed weights":  # ternary packs half the bytes: the same shape is in range
        assert call_gemm(fn="hq_gemm_w2a16", **kw) != hq.HQ_ERR_SHAPE
        assert call_gemm(fn="hq_gemm_w2a16", M=1, K=1 << 16, ldx=1 << 16, N=1 << 17, ldy=1 << 17) == hq.HQ_ERR_SHAPE


def test_range_limits_in_bias_fused_and_workspace_queries():
    L = hq.lib()
    # (The packed weights, K N / 2 or K N / 4 bytes, outgrow the scales and a bias, 2 or 4 K N /
    # group bytes, first for every group >= 32.)
    assert call_gemm(M=1, K=4096, N=1 << 26, ldy=1 << 26, bias=0x5000) == hq.HQ_ERR_SHAPE
    segs = (hq.Segment * 2)()
    segs[0] = hq.Segment(0x2000, 0x3000, None, 0x4000, 64, 64)
    segs[1] = hq.Segment(0x2000, 0x3000, None, 0x4000, 1 << 26, 1 << 26)
    assert L.hq_gemm_fused(0x1000, 1, 4096, 1, segs, 2, 1, 4096, 128, None, 0, None) == hq.HQ_ERR_SHAPE
    assert "segment 1" in L.hq_last_error().decode()
    assert L.hq_gemm_fused_noalloc(0x1000, 1, 4096, 1, segs, 2, 1, 4096, 128, None) == hq.HQ_ERR_SHAPE
    assert workspace_bytes(hq.FORMAT_INT4, 1, 1 << 16, 1 << 16)[0] == hq.HQ_ERR_SHAPE
    assert workspace_bytes(hq.FORMAT_TERNARY2, 1, 1 << 16, 1 << 16)[0] == hq.HQ_OK
    assert workspace_bytes(hq.FORMAT_INT4, 1 << 15, 1 << 15, 64)[0] == hq.HQ_ERR_SHAPE  # X: 2^31 bytes
    assert workspace_bytes_fused(hq.FORMAT_INT4, 1, 4096, [64, 1 << 26])[0] == hq.HQ_ERR_SHAPE


def test_bias_validation():
    assert call_gemm(bias=0x5002) == hq.HQ_ERR_ALIGNMENT
    segs = (hq.Segment * 1)()
    segs[0] = hq.Segment(0x2000, 0x3000, 0x5000, 0x4000, 64, 64)
    assert hq.lib().hq_gemm_fused(0x1000, 1, 4096, 2, segs, 1, 16, 4096, 128, None, 0, None) == hq.HQ_ERR_UNSUPPORTED
    assert "int4" in hq.lib().hq_last_error().decode()


def test_fused_rejects_bad_segments():
    L = hq.lib()
    segs = (hq.Segment * 9)()
    for i in range(9):
        segs[i] = hq.Segment(0x2000, 0x3000, None, 0x4000, 64, 64)
    assert L.hq_gemm_fused(0x1000, 1, 4096, 1, segs, 0, 16, 4096, 128, None, 0, None) == hq.HQ_ERR_INVALID_ARG
    assert L.hq_gemm_fused(0x1000, 1, 4096, 1, segs, 9, 16, 4096, 128, None, 0, None) == hq.HQ_ERR_INVALID_ARG
    assert L.hq_gemm_fused(0x1000, 1, 4096, 7, segs, 2, 16, 4096, 128, None, 0, None) == hq.HQ_ERR_INVALID_ARG
    segs[1] = hq.Segment(0x2000, 0x3000, None, 0x4000, 10, 64)
    assert L.hq_gemm_fused(0x1000, 1, 4096, 1, segs, 2, 16, 4096, 128, None, 0, None) == hq.HQ_ERR_SHAPE
    assert "segment 1" in L.hq_last_error().decode()


def test_last_error_is_per_thread():
    import threading

    assert call_gemm(M=0) == hq.HQ_ERR_SHAPE
    seen = {}

    def other():
        seen["msg"] = hq.lib().hq_last_error().decode()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == "" and hq.lib().hq_last_error().decode() != ""


def test_device_repack_rejects_bad_shapes():
    L = hq.lib()
    assert L.hq_repack_int4_device(0x1000, 0x2000, 100, 16, None) == hq.HQ_ERR_SHAPE
    assert L.hq_repack_ternary2_device(0, 0x2000, 128, 16, None, None) == hq.HQ_ERR_INVALID_ARG


# ---------------------------------------------------------------- host repacks
def test_repack_int4_ref_bit_exact_with_oracle():
    for K, N in [(32, 1), (128, 17), (4096, 64), (512, 300)]:
        src = O.gen_int4(5, 1, K, N)
        assert np.array_equal(hq.repack_int4_ref(src, K, N), O.repack_ref(src, K, N))


@pytest.mark.parametrize("K,N", [(128, 16), (128, 17), (256, 40), (1024, 3), (5120, 64)])
def test_int4_tile_layout_round_trip_and_to_ref(K, N):
    src = O.gen_int4(6, 1, K, N)
    packed = hq.repack(hq.FORMAT_INT4, src, K, N)
    assert packed.size == hq.packed_words(hq.FORMAT_INT4, K, N)
    back = hq.unpack(hq.FORMAT_INT4, packed, K, N)
    assert np.array_equal(back, src)
    # to_ref: the tile layout maps back to the reference "Marlin" layout bit for bit
    assert np.array_equal(hq.repack_int4_ref(back, K, N), O.repack_ref(src, K, N))


def test_int4_tile_layout_semantics():
    # Lane l of block (ct, kb), word c, element e: column 16*ct + l%16, k = 128*kb + 32*c + 8*(l//16) + e,
    # nibble position {0,4,1,5,2,6,3,7}[e].
    K, N = 256, 32
    q = np.random.default_rng(3).integers(0, 16, size=(K, N), dtype=np.uint32)
    lin = np.bitwise_or.reduce(q.reshape(K // 8, 8, N) << (4 * np.arange(8, dtype=np.uint32))[None, :, None], axis=1)
    packed = hq.repack(hq.FORMAT_INT4, lin.astype(np.uint32).ravel(), K, N).reshape(N // 16, K // 128, 64, 4)
    pos = [0, 4, 1, 5, 2, 6, 3, 7]
    for ct in range(N // 16):
        for kb in range(K // 128):
            for lane in (0, 5, 17, 63):
                for c in range(4):
                    for e in range(8):
                        k = 128 * kb + 32 * c + 8 * (lane // 16) + e
                        got = (packed[ct, kb, lane, c] >> (4 * pos[e])) & 0xF
                        assert got == q[k, 16 * ct + lane % 16]


def test_int4_padding_columns_decode_to_zero():
    K, N = 128, 20
    packed = hq.repack(hq.FORMAT_INT4, O.gen_int4(1, 1, K, N), K, N).reshape(2, 1, 64, 4)
    pad_lanes = [l for l in range(64) if 16 + l % 16 >= N]
    assert np.all(packed[1, 0, pad_lanes, :] == 0x88888888)


@pytest.mark.parametrize("K,N", [(128, 16), (256, 17), (512, 48), (5120, 40)])
def test_ternary_tile_layout_round_trip(K, N):
    src = O.gen_ternary(8, 1, K, N)
    packed = hq.repack(hq.FORMAT_TERNARY2, src, K, N)
    assert packed.size == hq.packed_words(hq.FORMAT_TERNARY2, K, N)
    assert np.array_equal(hq.unpack(hq.FORMAT_TERNARY2, packed, K, N), src)


def test_ternary_tile_layout_semantics():
    # (word << 2a) & 0xC000C000 must give the fp16/bf16 bits of 2t for elements (2h, 2h+1)
    # of chunk 2w + a//4 (a = 4*cw + h), lane column 16*ct + l%16.
    K, N = 256, 16
    t = np.random.default_rng(4).choice([-1, 0, 1], size=(K, N))
    c = (t + 1).astype(np.uint32)
    lin = np.bitwise_or.reduce(c.reshape(K // 16, 16, N) << (2 * np.arange(16, dtype=np.uint32))[None, :, None], axis=1)
    packed = hq.repack(hq.FORMAT_TERNARY2, lin.astype(np.uint32).ravel(), K, N).reshape(1, K // 128, 64, 2)
    val = {0x0000: 0, 0x4000: 2, 0xC000: -2}
    for kb in range(K // 128):
        for lane in range(64):
            for w in range(2):
                word = int(packed[0, kb, lane, w])
                for a in range(8):
                    v = ((word << (2 * a)) & 0xC000C000) & 0xFFFFFFFF
                    cw, h = divmod(a, 4)
                    chunk = 2 * w + cw
                    for half, e in ((v & 0xFFFF, 2 * h), (v >> 16, 2 * h + 1)):
                        k = 128 * kb + 32 * chunk + 8 * (lane // 16) + e
                        assert val[half] == 2 * t[k, lane % 16]


def test_ternary_repack_rejects_code_3():
    K, N = 128, 16
    src = O.gen_ternary(9, 1, K, N)
    src[3] |= 3 << 10
    with pytest.raises(hq.HQError) as ei:
        hq.repack(hq.FORMAT_TERNARY2, src, K, N)
    assert ei.value.status == hq.HQ_ERR_BAD_CODE


# ---------------------------------------------------------------- GGUF TQ1_0 import
def test_tq1_0_bytes():
    assert hq.tq1_0_bytes(5120, 27648) == 27648 * 20 * 56
    assert hq.tq1_0_bytes(128, 16) == 0 and hq.tq1_0_bytes(0, 16) == 0


@pytest.mark.parametrize("K,N", [(256, 1), (512, 17), (1280, 40)])
def test_convert_tq1_0_matches_oracle(K, N):
    blocks = O.gen_tq1_0(K + N, N, K, nonfinite_every=7)
    codes, scales = hq.convert_tq1_0(blocks, K, N)
    lin = codes.reshape(K // 16, N)
    for n in range(N):
        for b in range(K // 256):
            assert scales[b, n] == O.tq1_0_scale(blocks[n, b])
            c = O.tq1_0_codes(blocks[n, b])
            words = lin[16 * b:16 * (b + 1), n]
            mine = (words[:, None] >> (2 * np.arange(16, dtype=np.uint32))[None, :]) & 3
            assert np.array_equal(mine.reshape(256), c), (n, b)
    # The codes are valid ternary input: the host repack accepts them and round-trips.
    packed = hq.repack(hq.FORMAT_TERNARY2, codes, K, N)
    assert np.array_equal(hq.unpack(hq.FORMAT_TERNARY2, packed, K, N), codes)


def test_convert_tq1_0_rejects_bad_arguments():
    L = hq.lib()
    buf = np.zeros(1 << 16, dtype=np.uint8)
    p = buf.ctypes.data
    assert L.hq_convert_tq1_0(p, 128, 4, p, p) == hq.HQ_ERR_SHAPE
    assert L.hq_convert_tq1_0(None, 256, 4, p, p) == hq.HQ_ERR_INVALID_ARG
    assert L.hq_repack_tq1_0_device(p, 384, 4, p, p, None) == hq.HQ_ERR_SHAPE
    assert L.hq_repack_tq1_0_device(p + 4, 256, 4, p, p, None) == hq.HQ_ERR_ALIGNMENT


# ---------------------------------------------------------------- the int8 path
def test_int8_repack_layout_and_round_trip():
    rng = np.random.default_rng(5)
    K, N = 256, 37
    w = rng.integers(-128, 128, (K, N), dtype=np.int16).astype(np.int8)
    packed = hq.repack_int8(w)
    assert packed.size == hq.lib().hq_int8_packed_bytes(K, N) == K * 48
    assert np.array_equal(hq.unpack_int8(packed, K, N), w)
    # Byte of w[k][n]: tile (n // 16, k // 128) of 2 KiB, lane 16 ((k % 64) // 16) + n % 16 of 32
    # bytes, chunk (k % 128) // 64 of 16 bytes, element k % 16: each lane's 16 bytes are one
    # column's consecutive k, the B operand of v_mfma_i32_16x16x64_i8 (lane: column l % 16,
    # k-slice l / 16).
    for k, n in [(0, 0), (5, 3), (70, 17), (255, 36), (129, 20)]:
        off = ((n // 16) * (K // 128) + k // 128) * 2048 + (16 * ((k % 64) // 16) + n % 16) * 32 + ((k % 128) // 64) * 16 + k % 16
        assert packed[off] == w[k, n]
    # padding columns (37..47 of the last tile) are zero
    pad = packed.reshape(3, 2, 64, 32)[2][:, [l for l in range(64) if l % 16 >= 5], :]
    assert not pad.any()


def test_int8_shapes_and_workspace():
    L = hq.lib()
    assert L.hq_int8_packed_bytes(100, 16) == 0 and L.hq_int8_packed_bytes(128, 0) == 0
    b = ctypes.c_size_t(0)
    assert L.hq_workspace_bytes_w8a8(8, 5120, 27648, ctypes.byref(b)) == hq.HQ_OK and b.value >= 8 * 5120
    assert L.hq_workspace_bytes_w8a8(17, 5120, 512, ctypes.byref(b)) == hq.HQ_ERR_UNSUPPORTED
    assert L.hq_workspace_bytes_w8a8(4, 5000, 512, ctypes.byref(b)) == hq.HQ_ERR_SHAPE
    assert L.hq_workspace_bytes_w8a8(4, 262144, 512, ctypes.byref(b)) == hq.HQ_ERR_SHAPE  # int32 sum bound
    # argument checks before any launch
    assert L.hq_gemm_w8a8(None, 128, 0x1000, 0x2000, 0x3000, 16, 1, 128, 16, None, 0, None) == hq.HQ_ERR_INVALID_ARG
    assert L.hq_gemm_w8a8(0x1000, 100, 0x1000, 0x2000, 0x3000, 16, 1, 128, 16, None, 0, None) == hq.HQ_ERR_SHAPE
    assert L.hq_gemm_w8a8(0x1004, 128, 0x1000, 0x2000, 0x3000, 16, 1, 128, 16, None, 0, None) == hq.HQ_ERR_ALIGNMENT
    assert L.hq_gemm_w8a8(0x1000, 128, 0x1000, 0x2000, 0x3000, 16, 0, 128, 16, None, 0, None) == hq.HQ_ERR_UNSUPPORTED
    need = hq.workspace_bytes_w8a8(4, 1024, 64)
    assert L.hq_gemm_w8a8(0x1000, 1024, 0x1000, 0x2000, 0x3000, 64, 4, 1024, 64, 0x10000, need - 1, None) == \
        hq.HQ_ERR_WORKSPACE


@pytest.mark.parametrize("fmt,dt,M,slabs,sg", [
    (hq.FORMAT_INT4, hq.DTYPE_F16, 8, 256, 1), (hq.FORMAT_INT4, hq.DTYPE_F16, 8, 257, 2),
    (hq.FORMAT_INT4, hq.DTYPE_F16, 8, 383, 2), (hq.FORMAT_INT4, hq.DTYPE_F16, 8, 384, 2),
    (hq.FORMAT_INT4, hq.DTYPE_F16, 8, 512, 2), (hq.FORMAT_INT4, hq.DTYPE_F16, 8, 513, 3),
    (hq.FORMAT_INT4, hq.DTYPE_BF16, 1, 432, 2), (hq.FORMAT_INT4, hq.DTYPE_F16, 16, 432, 2),
    (hq.FORMAT_INT4, hq.DTYPE_F16, 16, 272, 2), (hq.FORMAT_TERNARY2, hq.DTYPE_BF16, 12, 320, 2),
    (hq.FORMAT_TERNARY2, hq.DTYPE_BF16, 8, 320, 1),
    (hq.FORMAT_TERNARY2, hq.DTYPE_BF16, 8, 432, 1), (hq.FORMAT_TERNARY2, hq.DTYPE_BF16, 9, 432, 2),
    (hq.FORMAT_INT4, hq.DTYPE_F16, 4, 544, 3), (hq.FORMAT_INT4, hq.DTYPE_F16, 16, 768, 3),
    (hq.FORMAT_INT4, hq.DTYPE_F16, 12, 769, 4), (hq.FORMAT_INT4, hq.DTYPE_BF16, 1, 864, 4),
    (hq.FORMAT_INT4, hq.DTYPE_F16, 16, 1024, 4), (hq.FORMAT_INT4, hq.DTYPE_F16, 4, 1025, 1),
    (hq.FORMAT_TERNARY2, hq.DTYPE_BF16, 4, 544, 3), (hq.FORMAT_TERNARY2, hq.DTYPE_BF16, 3, 640, 1),
    (hq.FORMAT_TERNARY2, hq.DTYPE_F16, 16, 640, 3), (hq.FORMAT_TERNARY2, hq.DTYPE_BF16, 1, 896, 4)])
def test_slab_groups_planned_by_slabs_per_cu(fmt, dt, M, slabs, sg):
    # The planner's rule on a 256-CU device (the count the library assumes without a device):
    # whole 4-tile slabs numbering 257..1024 run in groups of ceil(slabs / 256) per workgroup,
    # int4 at any M <= 16 (one or two rows may take 2-tile slabs first on a device), ternary in
    # pairs above eight rows, in triples from four rows, in quads at any row count; otherwise
    # one slab per workgroup.
    import torch

    if torch.cuda.is_available() and torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the boundaries are those of a 256-CU device")
    desc = hq.describe(fmt, dt, M, 5120, 64 * slabs)
    assert desc.startswith("hq_decode_xr_kernel<") or sg == 1, desc
    assert ",SG=" not in desc if sg == 1 else f",T=4,U=2,SG={sg}>" in desc, desc
    if sg > 1:
        assert f"workgroups={(slabs + sg - 1) // sg} of {sg} slabs ({slabs} slabs)" in desc, desc
        assert "x 1 pieces x 4 wavefronts" in desc, desc


@pytest.mark.parametrize("fmt,dt,M,K,N,want", [
    # few tiles (at most 128 on 256 CUs): one-tile slabs of eight wavefronts, whole up to 64
    # k-blocks, in ceil(k-blocks / 64) pieces beyond, more where the rows need them to fit
    (hq.FORMAT_INT4, hq.DTYPE_F16, 1, 5120, 1024, "T=1,U=4> workgroups=64 slabs x 1 pieces x 8 wavefronts"),
    (hq.FORMAT_INT4, hq.DTYPE_F16, 16, 5120, 1024, "T=1,U=4> workgroups=64 slabs x 1 pieces x 8 wavefronts"),
    (hq.FORMAT_TERNARY2, hq.DTYPE_BF16, 8, 5120, 2048, "T=1,U=4> workgroups=128 slabs x 1 pieces x 8 wavefronts"),
    (hq.FORMAT_INT4, hq.DTYPE_F16, 16, 8192, 1024, "T=1,U=4> workgroups=64 slabs x 2 pieces x 8 wavefronts"),
    (hq.FORMAT_INT4, hq.DTYPE_F16, 1, 27648, 1024, "T=1,U=4> workgroups=64 slabs x 4 pieces x 8 wavefronts"),
    (hq.FORMAT_INT4, hq.DTYPE_F16, 8, 27648, 512, "T=1,U=4> workgroups=32 slabs x 4 pieces x 8 wavefronts"),
    (hq.FORMAT_TERNARY2, hq.DTYPE_BF16, 16, 14336, 1024, "T=1,U=4> workgroups=64 slabs x 3 pieces x 8 wavefronts"),
    # ... unless no one-round grid of them exists (16 rows of K = 27648 need six pieces)
    (hq.FORMAT_INT4, hq.DTYPE_F16, 16, 27648, 1024, "hq_decode_ls_kernel<"),
    # 2-tile slabs two to a CU give way to 4-tile slabs one to a CU, of eight wavefronts
    (hq.FORMAT_INT4, hq.DTYPE_F16, 1, 4096, 14336, "T=4,U=2> workgroups=224 slabs x 1 pieces x 8 wavefronts"),
    (hq.FORMAT_TERNARY2, hq.DTYPE_BF16, 8, 4096, 11008, "T=4,U=2> workgroups=172 slabs x 1 pieces x 8 wavefronts"),
    # ... while 2-tile slabs one to a CU stay (5120 x 7168: 224 slabs)
    (hq.FORMAT_INT4, hq.DTYPE_F16, 4, 5120, 7168, "T=2,U=3> workgroups=224 slabs x 1 pieces x 8 wavefronts"),
    # ternary over a long K: K pieces also where the rows fit (int4 and a shorter K keep whole slabs)
    (hq.FORMAT_TERNARY2, hq.DTYPE_BF16, 1, 27648, 5120, "T=4,U=2> workgroups=80 slabs x 3 pieces x 8 wavefronts"),
    (hq.FORMAT_INT4, hq.DTYPE_F16, 1, 27648, 5120, "T=2,U=3> workgroups=160 slabs x 1 pieces x 8 wavefronts"),
    (hq.FORMAT_TERNARY2, hq.DTYPE_F16, 2, 17408, 5120, "T=2,U=3> workgroups=160 slabs x 1 pieces x 8 wavefronts"),
])
def test_decode_plans_by_tile_count(fmt, dt, M, K, N, want):
    # The planner's tile-count rules on a 256-CU device (the count the library assumes without
    # a device).
    import torch

    if torch.cuda.is_available() and torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the boundaries are those of a 256-CU device")
    desc = hq.describe(fmt, dt, M, K, N)
    assert want in desc, desc


@pytest.mark.parametrize("K,N,M,tiles", [(4096, 40960, 136, 480), (4096, 40960, 192, 480), (5120, 34816, 160, 408),
                                         (5120, 36864, 192, 432)])
def test_prefill_64_row_tiles_past_one_128_row_tile_per_cu(K, N, M, tiles):
    # 128-row tiles a few past one per CU (272-320 on 256 CUs) when 64-row tiles fit two per
    # CU: 64-row tiles (a rule on the CU count alone, not on the occupancy query).
    import torch

    if torch.cuda.is_available() and torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the boundaries are those of a 256-CU device")
    desc = hq.describe(hq.FORMAT_INT4, hq.DTYPE_F16, M, K, N)
    assert f"64-row tiles={tiles} whole={tiles}" in desc, desc
