"""ctypes binding of the CPU oracle (oracle/liboracle_hq.so) — test infrastructure only."""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE_DIR = ROOT / "oracle"
ORACLE_LIB = Path(os.environ.get("HQO_LIB", ORACLE_DIR / "liboracle_hq.so"))

F16, BF16 = 1, 2
INT4, TERNARY2 = 1, 2

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not ORACLE_LIB.exists():
        subprocess.run(["make", "-C", str(ORACLE_DIR), "-s"], check=True)
    L = ctypes.CDLL(str(ORACLE_LIB))
    u64, u32, u16, vp, sz, i32, dbl, f32 = (ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint16, ctypes.c_void_p,
                                             ctypes.c_size_t, ctypes.c_int, ctypes.c_double, ctypes.c_float)
    L.hqo_rng_u64.restype = u64
    L.hqo_rng_u64.argtypes = [u64, u64, u64]
    L.hqo_rng_uniform.restype = dbl
    L.hqo_rng_uniform.argtypes = [u64, u64, u64]
    L.hqo_gen_normal.argtypes = [u64, u64, dbl, i32, i32, vp, sz]
    L.hqo_gen_int4_linear.argtypes = [u64, u64, vp, u32, u32]
    L.hqo_gen_ternary2_linear.argtypes = [u64, u64, vp, u32, u32]
    L.hqo_f32_to_f16.restype = u16
    L.hqo_f32_to_f16.argtypes = [f32]
    L.hqo_f16_to_f32.restype = f32
    L.hqo_f16_to_f32.argtypes = [u16]
    L.hqo_f32_to_bf16.restype = u16
    L.hqo_f32_to_bf16.argtypes = [f32]
    L.hqo_bf16_to_f32.restype = f32
    L.hqo_bf16_to_f32.argtypes = [u16]
    L.hqo_to_f32.argtypes = [vp, i32, vp, sz]
    L.hqo_from_f32.argtypes = [vp, i32, vp, sz]
    L.hqo_repack_ref.argtypes = [vp, vp, u32, u32]
    L.hqo_dequant_int4.argtypes = [vp, vp, u32, u32, u32, vp]
    L.hqo_dequant_ternary2.restype = i32
    L.hqo_dequant_ternary2.argtypes = [vp, vp, u32, u32, u32, vp]
    L.hqo_gemm_f32.argtypes = [vp, vp, vp, u32, u32, u32, i32]
    L.hqo_qgemm.restype = i32
    L.hqo_qgemm.argtypes = [vp, i32, sz, i32, vp, vp, u32, u32, u32, u32, vp, i32]
    L.hqo_qgemm_bias.restype = i32
    L.hqo_qgemm_bias.argtypes = [vp, i32, sz, i32, vp, vp, vp, u32, u32, u32, u32, vp, i32]
    L.hqo_dequant_int4_bias.argtypes = [vp, vp, vp, u32, u32, u32, vp]
    L.hqo_fidelity.argtypes = [vp, vp, sz, ctypes.POINTER(dbl), ctypes.POINTER(dbl)]
    L.hqo_tq1_0_code.restype = u32
    L.hqo_tq1_0_code.argtypes = [vp, u32]
    L.hqo_tq1_0_scale.restype = u16
    L.hqo_tq1_0_scale.argtypes = [vp]
    L.hqo_gemv_tq1_0.argtypes = [vp, vp, vp, u32, u32, u32, i32]
    L.hqo_dequant_q4_k.argtypes = [vp, u32, u32, vp]
    L.hqo_int8_from_int4.argtypes = [vp, u32, u32, vp]
    L.hqo_quantize_x_int8.argtypes = [f32]
    L.hqo_quantize_x_int8.restype = ctypes.c_int8
    L.hqo_gemm_int8.argtypes = [vp, sz, vp, vp, u32, u32, u32, vp, i32]
    _lib = L
    return L


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data


def gen_normal(seed: int, stream: int, n: int, sigma: float = 1.0, absval: bool = False, dtype: int = F16) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().hqo_gen_normal(seed, stream, sigma, int(absval), dtype, _p(out), n)
    return out


def gen_int4(seed: int, stream: int, K: int, N: int) -> np.ndarray:
    out = np.empty((K // 8) * N, dtype=np.uint32)
    lib().hqo_gen_int4_linear(seed, stream, _p(out), K, N)
    return out


def gen_ternary(seed: int, stream: int, K: int, N: int) -> np.ndarray:
    out = np.empty((K // 16) * N, dtype=np.uint32)
    lib().hqo_gen_ternary2_linear(seed, stream, _p(out), K, N)
    return out


def to_f32(bits: np.ndarray, dtype: int) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    lib().hqo_to_f32(_p(bits), dtype, _p(out), bits.size)
    return out


def from_f32(x: np.ndarray, dtype: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().hqo_from_f32(_p(x), dtype, _p(out), x.size)
    return out


def repack_ref(linear: np.ndarray, K: int, N: int) -> np.ndarray:
    src = np.ascontiguousarray(linear, dtype=np.uint32)
    dst = np.empty(src.size, dtype=np.uint32)
    lib().hqo_repack_ref(_p(src), _p(dst), K, N)
    return dst


def dequant(fmt: int, linear: np.ndarray, scales: np.ndarray, K: int, N: int, group: int,
            out: np.ndarray | None = None) -> np.ndarray:
    w = np.ascontiguousarray(linear, dtype=np.uint32)
    s = np.ascontiguousarray(scales, dtype=np.uint16)
    if out is None:
        out = np.empty((K, N), dtype=np.float32)
    assert out.shape == (K, N) and out.dtype == np.float32 and out.flags["C_CONTIGUOUS"]
    if fmt == INT4:
        lib().hqo_dequant_int4(_p(w), _p(s), K, N, group, _p(out))
    else:
        if lib().hqo_dequant_ternary2(_p(w), _p(s), K, N, group, _p(out)) != 0:
            raise ValueError("ternary code 3 in weight")
    return out


def dequant_int4_bias(linear: np.ndarray, scales: np.ndarray, bias: np.ndarray | None, K: int, N: int,
                      group: int) -> np.ndarray:
    """The reference's host dequantisation w = q * s + b with a caller bias (fp32 [K/group, N])."""
    w = np.ascontiguousarray(linear, dtype=np.uint32)
    s = np.ascontiguousarray(scales, dtype=np.uint16)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    out = np.empty((K, N), dtype=np.float32)
    lib().hqo_dequant_int4_bias(_p(w), _p(s), None if b is None else _p(b), K, N, group, _p(out))
    return out


def gemm_f32(X: np.ndarray, W: np.ndarray, threads: int = 8) -> np.ndarray:
    X = np.ascontiguousarray(X, dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.float32)
    M, K = X.shape
    K2, N = W.shape
    assert K == K2
    Y = np.empty((M, N), dtype=np.float32)
    lib().hqo_gemm_f32(_p(X), _p(W), _p(Y), M, K, N, threads)
    return Y


def qgemm(fmt: int, X_bits: np.ndarray, xdtype: int, linear: np.ndarray, scales: np.ndarray, N: int,
          group: int = 128, threads: int = 8) -> np.ndarray:
    """Reference dequantize-then-matmul: fp32 Y[M, N] from fp16/bf16 activation bits [M, K]."""
    X = np.ascontiguousarray(X_bits, dtype=np.uint16)
    M, K = X.shape
    w = np.ascontiguousarray(linear, dtype=np.uint32)
    s = np.ascontiguousarray(scales, dtype=np.uint16)
    Y = np.empty((M, N), dtype=np.float32)
    rc = lib().hqo_qgemm(_p(X), xdtype, K, fmt, _p(w), _p(s), M, K, N, group, _p(Y), threads)
    if rc == -1:
        raise ValueError("ternary code 3 in weight")
    if rc != 0:
        raise MemoryError("oracle allocation failed")
    return Y


def qgemm_bias(X_bits: np.ndarray, xdtype: int, linear: np.ndarray, scales: np.ndarray, bias: np.ndarray | None,
               N: int, group: int = 128, threads: int = 8) -> np.ndarray:
    """qgemm for int4 weights with the reference's bias: w = q * s + b (b fp32 [K/group, N])."""
    X = np.ascontiguousarray(X_bits, dtype=np.uint16)
    M, K = X.shape
    w = np.ascontiguousarray(linear, dtype=np.uint32)
    s = np.ascontiguousarray(scales, dtype=np.uint16)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    Y = np.empty((M, N), dtype=np.float32)
    rc = lib().hqo_qgemm_bias(_p(X), xdtype, K, INT4, _p(w), _p(s), None if b is None else _p(b), M, K, N, group,
                              _p(Y), threads)
    if rc != 0:
        raise MemoryError("oracle allocation failed")
    return Y


def fidelity(a: np.ndarray, b: np.ndarray) -> tuple[float, float]:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    mx, mse = ctypes.c_double(), ctypes.c_double()
    lib().hqo_fidelity(_p(a), _p(b), a.size, ctypes.byref(mx), ctypes.byref(mse))
    return mx.value, mse.value


TQ1_0_BLOCK_BYTES = 56


def tq1_0_codes(block: np.ndarray) -> np.ndarray:
    """Codes c = t + 1 of the 256 elements of one 56-byte TQ1_0 block."""
    b = np.ascontiguousarray(block, dtype=np.uint8)
    assert b.size == TQ1_0_BLOCK_BYTES
    return np.array([lib().hqo_tq1_0_code(_p(b), i) for i in range(256)], dtype=np.uint32)


def tq1_0_scale(block: np.ndarray) -> int:
    b = np.ascontiguousarray(block, dtype=np.uint8)
    return int(lib().hqo_tq1_0_scale(_p(b)))


def gemv_tq1_0(X: np.ndarray, blocks: np.ndarray, N: int, threads: int = 8) -> np.ndarray:
    """kernel_gemv_tq1_0 over the rows of X (fp32 [M, K]); blocks: N rows of K/256 blocks."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    W = np.ascontiguousarray(blocks, dtype=np.uint8)
    M, K = X.shape
    assert W.size == N * (K // 256) * TQ1_0_BLOCK_BYTES
    Y = np.empty((M, N), dtype=np.float32)
    lib().hqo_gemv_tq1_0(_p(X), _p(W), _p(Y), M, K, N, threads)
    return Y


def gen_tq1_0(seed: int, N: int, K: int, nonfinite_every: int = 0) -> np.ndarray:
    """Random TQ1_0 blocks [N][K/256][56] (bytes uniform on 0..255, so every byte value, also those
    above 242 that no encoder writes, is exercised); d = |N(0, 0.02)| in fp16; with nonfinite_every
    > 0, every such block gets an Inf or NaN d."""
    nb = K // 256
    raw = np.random.default_rng(seed).integers(0, 256, N * nb * TQ1_0_BLOCK_BYTES, dtype=np.uint8)
    blocks = raw.reshape(N * nb, TQ1_0_BLOCK_BYTES)
    d = gen_normal(seed, 12, N * nb, 0.02, True, F16)
    if nonfinite_every:
        d[::nonfinite_every] = 0x7C00  # +Inf
        d[nonfinite_every // 2::nonfinite_every] = 0x7E00  # NaN
    blocks[:, 0] = (d & 0xFF).astype(np.uint8)
    blocks[:, 1] = (d >> 8).astype(np.uint8)
    return blocks.reshape(N, nb, TQ1_0_BLOCK_BYTES)


# ------------------------------------------------------------ problem builder
class Problem:
    """Seeded synthetic inputs of one qGEMM case (the distributions of the benchmark configs).
    bias: None (zero point 8), "random" (fp32 bias -8 s + N(0, 0.02) per group and column: the
    weight of code 8 becomes a small random offset) or "minus8s" (exactly -8 s, the reference's
    own data)."""

    def __init__(self, fmt: int, M: int, K: int, N: int, group: int = 128, xdtype: int = F16, seed: int = 42,
                 x_sigma: float = 1.0, s_sigma: float = 0.02, bias: str | None = None):
        self.fmt, self.M, self.K, self.N, self.group, self.xdtype, self.seed = fmt, M, K, N, group, xdtype, seed
        self.X = gen_normal(seed, 1, M * K, x_sigma, False, xdtype).reshape(M, K)
        self.scales = gen_normal(seed, 2, (K // group) * N, s_sigma, True, F16).reshape(K // group, N)
        self.W = gen_int4(seed, 3, K, N) if fmt == INT4 else gen_ternary(seed, 3, K, N)
        self.bias = None
        if bias is not None:
            s32 = to_f32(self.scales, F16)
            self.bias = (-8.0 * s32).astype(np.float32)
            if bias == "random":
                off = to_f32(gen_normal(seed, 4, (K // group) * N, 0.02, False, F16), F16).reshape(K // group, N)
                self.bias = (self.bias + off).astype(np.float32)

    def reference(self, rows=None, threads: int = 8) -> np.ndarray:
        X = self.X if rows is None else self.X[rows]
        if self.bias is not None:
            return qgemm_bias(X, self.xdtype, self.W, self.scales, self.bias, self.N, self.group, threads)
        return qgemm(self.fmt, X, self.xdtype, self.W, self.scales, self.N, self.group, threads)


def normwise_error(y: np.ndarray, r: np.ndarray) -> float:
    """max |y - r| / max |r| — the acceptance metric (tolerance 1e-2)."""
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    denom = np.max(np.abs(r))
    return float(np.max(np.abs(y - r)) / denom) if denom > 0 else float(np.max(np.abs(y - r)))


def elementwise_error(y: np.ndarray, r: np.ndarray, floor_frac: float = 1e-2) -> tuple[float, int]:
    """max |y - r| / |r| over |r| >= floor_frac * rms(r), and how many elements fall below the floor."""
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    floor = floor_frac * np.sqrt(np.mean(r * r))
    m = np.abs(r) >= floor
    rel = np.abs(y[m] - r[m]) / np.abs(r[m]) if m.any() else np.zeros(1)
    return float(rel.max()), int((~m).sum())


Q4_K_BLOCK_BYTES = 144


def dequant_q4_k(blocks: np.ndarray, K: int, N: int) -> np.ndarray:
    """GGML Q4_K blocks (N rows of K/256 blocks) -> fp32 Wdq [K, N] (the published dequantisation)."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    assert b.size == N * (K // 256) * Q4_K_BLOCK_BYTES
    out = np.empty((K, N), dtype=np.float32)
    lib().hqo_dequant_q4_k(_p(b), K, N, _p(out))
    return out


# ---------------------------------------------------------------- the int8 path
def int8_from_int4(linear: np.ndarray, K: int, N: int) -> np.ndarray:
    """int8 [K][N] weights q * 16 - 128 of the int4 codes (marlin_gemm.cu:508)."""
    out = np.empty((K, N), dtype=np.int8)
    lib().hqo_int8_from_int4(_p(np.ascontiguousarray(linear, dtype=np.uint32)), K, N, _p(out))
    return out


def quantize_x_int8(x: float) -> int:
    return int(lib().hqo_quantize_x_int8(float(x)))


def gemm_int8(X: np.ndarray, W: np.ndarray, scales: np.ndarray, threads: int = 8) -> np.ndarray:
    """kernel_cutlass_int8_gemm (marlin_gemm.cu:327-377): X fp32 [M][K], W int8 [K][N], scales fp32 [N]."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    M, K = X.shape
    N = W.shape[1]
    Y = np.empty((M, N), dtype=np.float32)
    lib().hqo_gemm_int8(_p(X), K, _p(W), _p(scales), M, K, N, _p(Y), threads)
    return Y
