"""ctypes binding of libnebula_hq.so (include/hq_qgemm.h) with torch/numpy helpers.

torch supplies device memory and streams only; every computation runs in the HIP
library. If the library is missing this module raises on first use: there is no
fallback path.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

_PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("HQ_LIB", _PKG / "lib" / "libnebula_hq.so"))

HQ_OK = 0
HQ_ERR_INVALID_ARG = 1
HQ_ERR_SHAPE = 2
HQ_ERR_ALIGNMENT = 3
HQ_ERR_UNSUPPORTED = 4
HQ_ERR_WORKSPACE = 5
HQ_ERR_BAD_CODE = 6
HQ_ERR_DEVICE = 7
HQ_ERR_INTERNAL = 8
HQ_ERR_FORMAT = 9
HQ_ERR_NOT_FOUND = 10
HQ_ERR_IO = 11

DTYPE_F16 = 1
DTYPE_BF16 = 2
FORMAT_INT4 = 1
FORMAT_TERNARY2 = 2
MAX_SEGMENTS = 8
NOALLOC_SCRATCH_BYTES = 16 << 20  # HQ_NOALLOC_SCRATCH_BYTES

# Every symbol include/hq_qgemm.h declares.
EXPORTS = (
    "hq_version", "hq_last_error", "hq_status_string", "hq_linear_words", "hq_packed_words",
    "hq_workspace_bytes", "hq_workspace_bytes_fused", "hq_describe_gemm", "hq_device_status", "hq_repack_int4_ref", "hq_repack_int4", "hq_repack_ternary2",
    "hq_unpack_int4", "hq_unpack_ternary2", "hq_repack_int4_device", "hq_repack_ternary2_device",
    "hq_gemm_w4a16", "hq_gemm_w2a16", "hq_gemm_fused", "hq_gemm_fused_noalloc", "hq_tq1_0_bytes", "hq_convert_tq1_0",
    "hq_repack_tq1_0_device", "hq_gguf_open", "hq_gguf_parse", "hq_gguf_close", "hq_gguf_header",
    "hq_gguf_tensor_at", "hq_gguf_find_tensor", "hq_gguf_get_int", "hq_gguf_get_float", "hq_gguf_get_string",
    "hq_gguf_get_array", "hq_gguf_load_tq1_0", "hq_convert_q4_k", "hq_gguf_convert_q4_k",
    "hq_int8_packed_bytes", "hq_repack_int8", "hq_unpack_int8", "hq_workspace_bytes_w8a8", "hq_gemm_w8a8",
)


class HQError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"hq status {status}: {message}")
        self.status = status
        self.message = message


class Segment(ctypes.Structure):
    _fields_ = [
        ("Wp", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("Y", ctypes.c_void_p),
        ("ldy", ctypes.c_int64),
        ("N", ctypes.c_uint32),
    ]


_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """Load the HIP library (fails loudly if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: run `python -m nebula_amd.build` (or __graft_entry__.build())")
    L = ctypes.CDLL(str(LIB_PATH))
    u32, i64, sz, vp, i32 = ctypes.c_uint32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int
    L.hq_version.restype = ctypes.c_char_p
    L.hq_last_error.restype = ctypes.c_char_p
    L.hq_status_string.restype = ctypes.c_char_p
    L.hq_status_string.argtypes = [i32]
    L.hq_linear_words.restype = sz
    L.hq_linear_words.argtypes = [i32, u32, u32]
    L.hq_packed_words.restype = sz
    L.hq_packed_words.argtypes = [i32, u32, u32]
    L.hq_workspace_bytes.restype = i32
    L.hq_workspace_bytes.argtypes = [i32, u32, u32, u32, u32, ctypes.POINTER(sz)]
    L.hq_workspace_bytes_fused.restype = i32
    L.hq_workspace_bytes_fused.argtypes = [i32, u32, u32, u32, ctypes.POINTER(u32), u32, i32, ctypes.POINTER(sz)]
    L.hq_describe_gemm.restype = i32
    L.hq_describe_gemm.argtypes = [i32, i32, u32, u32, u32, u32, i32, ctypes.c_char_p, sz]
    L.hq_device_status.restype = i32
    L.hq_device_status.argtypes = [vp]
    for name in ("hq_repack_int4_ref", "hq_repack_int4", "hq_repack_ternary2", "hq_unpack_int4", "hq_unpack_ternary2"):
        f = getattr(L, name)
        f.restype = i32
        f.argtypes = [vp, vp, u32, u32]
    L.hq_repack_int4_device.restype = i32
    L.hq_repack_int4_device.argtypes = [vp, vp, u32, u32, vp]
    L.hq_repack_ternary2_device.restype = i32
    L.hq_repack_ternary2_device.argtypes = [vp, vp, u32, u32, vp, vp]
    L.hq_gemm_w4a16.restype = i32
    L.hq_gemm_w4a16.argtypes = [vp, i32, i64, vp, vp, vp, vp, i64, u32, u32, u32, u32, vp, sz, vp]
    L.hq_gemm_w2a16.restype = i32
    L.hq_gemm_w2a16.argtypes = [vp, i32, i64, vp, vp, vp, i64, u32, u32, u32, u32, vp, sz, vp]
    L.hq_tq1_0_bytes.restype = sz
    L.hq_tq1_0_bytes.argtypes = [u32, u32]
    L.hq_convert_tq1_0.restype = i32
    L.hq_convert_tq1_0.argtypes = [vp, u32, u32, vp, vp]
    L.hq_repack_tq1_0_device.restype = i32
    L.hq_repack_tq1_0_device.argtypes = [vp, u32, u32, vp, vp, vp]
    L.hq_gemm_fused.restype = i32
    L.hq_gemm_fused.argtypes = [vp, i32, i64, i32, ctypes.POINTER(Segment), u32, u32, u32, u32, vp, sz, vp]
    L.hq_gemm_fused_noalloc.restype = i32
    L.hq_gemm_fused_noalloc.argtypes = [vp, i32, i64, i32, ctypes.POINTER(Segment), u32, u32, u32, u32, vp]
    L.hq_int8_packed_bytes.restype = sz
    L.hq_int8_packed_bytes.argtypes = [u32, u32]
    for f in (L.hq_repack_int8, L.hq_unpack_int8):
        f.restype = i32
        f.argtypes = [vp, u32, u32, vp]
    L.hq_workspace_bytes_w8a8.restype = i32
    L.hq_workspace_bytes_w8a8.argtypes = [u32, u32, u32, ctypes.POINTER(sz)]
    L.hq_gemm_w8a8.restype = i32
    L.hq_gemm_w8a8.argtypes = [vp, i64, vp, vp, vp, i64, u32, u32, u32, vp, sz, vp]
    _lib = L
    return L


def check(status: int) -> None:
    if status != HQ_OK:
        raise HQError(status, lib().hq_last_error().decode())


def version() -> str:
    return lib().hq_version().decode()


def linear_words(fmt: int, K: int, N: int) -> int:
    return int(lib().hq_linear_words(fmt, K, N))


def packed_words(fmt: int, K: int, N: int) -> int:
    return int(lib().hq_packed_words(fmt, K, N))


def _u32(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype != np.uint32:
        a = a.view(np.uint32) if a.dtype.itemsize == 4 else a.astype(np.uint32)
    return a


# ---------------------------------------------------------------- host repacks
def repack_int4_ref(linear: np.ndarray, K: int, N: int) -> np.ndarray:
    src = _u32(linear)
    if src.size != (K // 8) * N:
        raise ValueError(f"linear weight has {src.size} words, expected {(K // 8) * N}")
    dst = np.empty((K // 8) * N, dtype=np.uint32)
    check(lib().hq_repack_int4_ref(src.ctypes.data, dst.ctypes.data, K, N))
    return dst


def repack(fmt: int, linear: np.ndarray, K: int, N: int) -> np.ndarray:
    src = _u32(linear)
    if src.size != linear_words(fmt, K, N):
        raise ValueError(f"linear weight has {src.size} words, expected {linear_words(fmt, K, N)}")
    dst = np.empty(max(packed_words(fmt, K, N), 1), dtype=np.uint32)
    f = lib().hq_repack_int4 if fmt == FORMAT_INT4 else lib().hq_repack_ternary2
    check(f(src.ctypes.data, dst.ctypes.data, K, N))
    return dst


def unpack(fmt: int, packed: np.ndarray, K: int, N: int) -> np.ndarray:
    src = _u32(packed)
    if src.size < packed_words(fmt, K, N):
        raise ValueError(f"packed weight has {src.size} words, expected {packed_words(fmt, K, N)}")
    dst = np.empty(linear_words(fmt, K, N), dtype=np.uint32)
    f = lib().hq_unpack_int4 if fmt == FORMAT_INT4 else lib().hq_unpack_ternary2
    check(f(src.ctypes.data, dst.ctypes.data, K, N))
    return dst


def tq1_0_bytes(K: int, N: int) -> int:
    return int(lib().hq_tq1_0_bytes(K, N))


def convert_tq1_0(blocks: np.ndarray, K: int, N: int) -> tuple[np.ndarray, np.ndarray]:
    """GGUF TQ1_0 blocks (N rows of K/256 56-byte blocks) -> (ternary linear codes [K/16 * N] u32,
    fp16 scale bits [K/256, N] u16); use the scales with group = 256."""
    src = np.ascontiguousarray(blocks, dtype=np.uint8)
    if src.size != tq1_0_bytes(K, N):
        raise ValueError(f"TQ1_0 tensor has {src.size} bytes, expected {tq1_0_bytes(K, N)}")
    codes = np.empty(linear_words(FORMAT_TERNARY2, K, N), dtype=np.uint32)
    scales = np.empty((K // 256, N), dtype=np.uint16)
    check(lib().hq_convert_tq1_0(src.ctypes.data, K, N, codes.ctypes.data, scales.ctypes.data))
    return codes, scales


# ---------------------------------------------------------------- device calls
def _stream_ptr(stream) -> Optional[int]:
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _dt(t) -> int:
    import torch

    if t.dtype == torch.float16:
        return DTYPE_F16
    if t.dtype == torch.bfloat16:
        return DTYPE_BF16
    raise TypeError(f"activations must be float16 or bfloat16, got {t.dtype}")


def repack_device(fmt: int, linear, K: int, N: int, stream=None, bad_flag=None):
    """Repack a device tensor of linear words (int32/uint32 view) into a new device tensor."""
    import torch

    if not linear.is_cuda or not linear.is_contiguous() or linear.element_size() != 4:
        raise ValueError("linear weight must be a contiguous 32-bit device tensor")
    if linear.numel() != linear_words(fmt, K, N):
        raise ValueError(f"linear weight has {linear.numel()} words, expected {linear_words(fmt, K, N)}")
    out = torch.empty(packed_words(fmt, K, N), dtype=torch.int32, device=linear.device)
    sp = _stream_ptr(stream)
    if fmt == FORMAT_INT4:
        check(lib().hq_repack_int4_device(linear.data_ptr(), out.data_ptr(), K, N, sp))
    else:
        flag = bad_flag.data_ptr() if bad_flag is not None else None
        check(lib().hq_repack_ternary2_device(linear.data_ptr(), out.data_ptr(), K, N, flag, sp))
    return out


def repack_tq1_0_device(blocks, K: int, N: int, stream=None, out=None):
    """GGUF TQ1_0 blocks in a device uint8 tensor -> (packed ternary weight, fp16 scales [K/256, N]),
    device tensors (new ones, or the pair `out`); use them with FORMAT_TERNARY2 and group = 256."""
    import torch

    if blocks.numel() * blocks.element_size() != tq1_0_bytes(K, N):
        raise ValueError(f"TQ1_0 tensor has {blocks.numel() * blocks.element_size()} bytes, "
                         f"expected {tq1_0_bytes(K, N)}")
    if out is None:
        packed = torch.empty(packed_words(FORMAT_TERNARY2, K, N), dtype=torch.int32, device=blocks.device)
        scales = torch.empty((K // 256, N), dtype=torch.float16, device=blocks.device)
    else:
        packed, scales = out
        if packed.numel() * packed.element_size() < 4 * packed_words(FORMAT_TERNARY2, K, N) or \
                scales.numel() * scales.element_size() < 2 * (K // 256) * N:
            raise ValueError("output tensors too small")
    check(lib().hq_repack_tq1_0_device(blocks.data_ptr(), K, N, packed.data_ptr(), scales.data_ptr(),
                                       _stream_ptr(stream)))
    return packed, scales


def workspace_bytes(fmt: int, M: int, K: int, N: int, group: int = 128) -> int:
    """Bytes of the fix-up workspace for this shape on the current device (0: none); covers calls
    with and without a bias."""
    b = ctypes.c_size_t(0)
    check(lib().hq_workspace_bytes(fmt, M, K, N, group, ctypes.byref(b)))
    return int(b.value)


def workspace_bytes_fused(fmt: int, M: int, K: int, Ns: Sequence[int], group: int = 128, with_bias: bool = False) -> int:
    """Exactly the workspace one fused call over segments of widths Ns asks for."""
    arr = (ctypes.c_uint32 * len(Ns))(*Ns)
    b = ctypes.c_size_t(0)
    check(lib().hq_workspace_bytes_fused(fmt, M, K, group, arr, len(Ns), int(with_bias), ctypes.byref(b)))
    return int(b.value)


def describe(fmt: int, dtype: int, M: int, K: int, N: int, group: int = 128, with_bias: bool = False) -> str:
    """The plan (kernel, tiling, grid) a call of this shape runs on the current device."""
    buf = ctypes.create_string_buffer(512)
    check(lib().hq_describe_gemm(fmt, dtype, M, K, N, group, int(with_bias), buf, len(buf)))
    return buf.value.decode()


def device_status(stream=None) -> None:
    """Wait for the stream, then raise HQError if a kernel reported a fault (a bounded wait that
    gave up) since the last check."""
    check(lib().hq_device_status(_stream_ptr(stream)))


def _ws(workspace):
    """(pointer, bytes) of a caller workspace tensor (zero-filled before first use), or (None, 0)."""
    if workspace is None:
        return None, 0
    if not workspace.is_cuda or not workspace.is_contiguous():
        raise ValueError("workspace must be a contiguous device tensor")
    return workspace.data_ptr(), workspace.numel() * workspace.element_size()


def _nbytes(t) -> int:
    return t.numel() * t.element_size()


def _check_rows(name: str, t, rows: int, cols: int, dtype) -> None:
    """t must be a device matrix of at least rows x cols elements of dtype, unit column stride."""
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    if t.dtype != dtype:
        raise ValueError(f"{name} has dtype {t.dtype}, expected {dtype}")
    if t.shape[0] < rows or t.shape[1] < cols:
        raise ValueError(f"{name} has shape {tuple(t.shape)}, needs at least ({rows}, {cols})")
    if t.stride(1) != 1 and t.shape[1] > 1:
        raise ValueError(f"{name} must have unit stride along its last dimension, got strides {t.stride()}")
    if t.shape[0] > 1 and t.stride(0) < cols:
        raise ValueError(f"{name} rows overlap: stride {t.stride(0)} < {cols}")


def _check_weight(fmt: int, Wp, scales, bias, K: int, N: int, group: int, X) -> None:
    import torch

    if not (Wp.is_cuda and scales.is_cuda) or Wp.device != X.device or scales.device != X.device:
        raise ValueError("Wp and scales must be device tensors on X's device")
    if not (Wp.is_contiguous() and scales.is_contiguous()):
        raise ValueError("Wp and scales must be contiguous")
    if group <= 0 or K % group:
        raise ValueError(f"K={K} must be a multiple of group={group}")
    need_w = 4 * packed_words(fmt, K, N)
    if _nbytes(Wp) < need_w:
        raise ValueError(f"packed weight has {_nbytes(Wp)} bytes, K={K} N={N} needs {need_w}")
    if scales.element_size() != 2 or scales.numel() < (K // group) * N:
        raise ValueError(f"scales must hold at least {(K // group) * N} fp16 values")
    if bias is not None:
        if fmt != FORMAT_INT4:
            raise ValueError("a bias is supported for int4 weights only")
        if not bias.is_cuda or bias.device != X.device or bias.dtype != torch.float32 or not bias.is_contiguous():
            raise ValueError("bias must be a contiguous float32 device tensor on X's device")
        if bias.numel() < (K // group) * N:
            raise ValueError(f"bias must hold at least {(K // group) * N} values")


def gemm(fmt: int, X, Wp, scales, N: int, group: int = 128, out=None, stream=None, workspace=None, bias=None):
    """Y[M, N] = X[M, K] @ dequant(Wp) with fp32 accumulation (Y in X's dtype).

    dequant: int4 (q - 8) * scale, or q * scale + bias with a float32 bias [K/group, N];
    ternary t * scale. workspace: optional device tensor of at least workspace_bytes() bytes,
    zero-filled before its first use; by default the library's own per-stream buffer is used.
    Shapes, dtypes, devices and strides are checked here: the kernels size their buffer
    descriptors from the shape, not from the allocations."""
    import torch

    M, K = X.shape
    _check_rows("X", X, M, K, X.dtype)
    _dt(X)
    _check_weight(fmt, Wp, scales, bias, K, N, group, X)
    if out is None:
        out = torch.empty((M, N), dtype=X.dtype, device=X.device)
    _check_rows("out", out, M, N, X.dtype)
    if out.device != X.device:
        raise ValueError("out must be on X's device")
    wp, wb = _ws(workspace)
    L = lib()
    if fmt == FORMAT_INT4:
        st = L.hq_gemm_w4a16(X.data_ptr(), _dt(X), X.stride(0), Wp.data_ptr(), scales.data_ptr(),
                             bias.data_ptr() if bias is not None else None, out.data_ptr(), out.stride(0),
                             M, K, N, group, wp, wb, _stream_ptr(stream))
    else:
        if bias is not None:
            raise ValueError("a bias is supported for int4 weights only")
        st = L.hq_gemm_w2a16(X.data_ptr(), _dt(X), X.stride(0), Wp.data_ptr(), scales.data_ptr(), out.data_ptr(),
                             out.stride(0), M, K, N, group, wp, wb, _stream_ptr(stream))
    check(st)
    return out


def gemm_fused(fmt: int, X, segments: Sequence[tuple], group: int = 128, outs=None, stream=None, workspace=None,
               noalloc: bool = False):
    """segments: (Wp, scales, N) or (Wp, scales, N, bias) per projection; returns one output per
    segment. noalloc: run hq_gemm_fused_noalloc (its workspace is the library's static scratch;
    `outs` must then be given by a caller that cannot allocate)."""
    import torch

    M, K = X.shape
    _check_rows("X", X, M, K, X.dtype)
    _dt(X)
    if not 1 <= len(segments) <= MAX_SEGMENTS:
        raise ValueError(f"need 1..{MAX_SEGMENTS} segments, got {len(segments)}")
    if outs is None:
        outs = [torch.empty((M, seg[2]), dtype=X.dtype, device=X.device) for seg in segments]
    if len(outs) != len(segments):
        raise ValueError("one output per segment")
    arr = (Segment * len(segments))()
    for i, (seg, y) in enumerate(zip(segments, outs)):
        wp, sc, n = seg[:3]
        b = seg[3] if len(seg) > 3 else None
        _check_weight(fmt, wp, sc, b, K, n, group, X)
        _check_rows(f"outs[{i}]", y, M, n, X.dtype)
        arr[i] = Segment(wp.data_ptr(), sc.data_ptr(), b.data_ptr() if b is not None else None, y.data_ptr(),
                         y.stride(0), n)
    if noalloc:
        if workspace is not None:
            raise ValueError("noalloc calls use the library's static scratch, not a workspace")
        check(lib().hq_gemm_fused_noalloc(X.data_ptr(), _dt(X), X.stride(0), fmt, arr, len(segments), M, K, group,
                                          _stream_ptr(stream)))
        return outs
    wp, wb = _ws(workspace)
    check(lib().hq_gemm_fused(X.data_ptr(), _dt(X), X.stride(0), fmt, arr, len(segments), M, K, group, wp, wb,
                              _stream_ptr(stream)))
    return outs


# ---------------------------------------------------------------- the int8 path
def repack_int8(w_kn: np.ndarray) -> np.ndarray:
    """int8 weights [K][N] -> the gfx950 int8 tile layout (hq_int8_packed_bytes(K, N) int8)."""
    w_kn = np.ascontiguousarray(w_kn, dtype=np.int8)
    K, N = w_kn.shape
    out = np.empty(lib().hq_int8_packed_bytes(K, N), dtype=np.int8)
    if out.size == 0:
        raise ValueError(f"K={K} must be a positive multiple of 128 and N >= 1")
    check(lib().hq_repack_int8(w_kn.ctypes.data, K, N, out.ctypes.data))
    return out


def unpack_int8(packed: np.ndarray, K: int, N: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.int8)
    if packed.size != lib().hq_int8_packed_bytes(K, N):
        raise ValueError("packed size does not match K, N")
    out = np.empty((K, N), dtype=np.int8)
    check(lib().hq_unpack_int8(packed.ctypes.data, K, N, out.ctypes.data))
    return out


def workspace_bytes_w8a8(M: int, K: int, N: int) -> int:
    b = ctypes.c_size_t(0)
    check(lib().hq_workspace_bytes_w8a8(M, K, N, ctypes.byref(b)))
    return b.value


def gemm_w8a8(X, Wp, scales, N: int, out=None, stream=None, workspace=None):
    """The int8 path: Y[M, N] (fp32) = scales[n] * sum_k int8(clamp(127 X)) W / 127, X fp32 [M, K]
    (M <= 16), Wp the int8 tile layout (repack_int8) on X's device, scales fp32 [N]."""
    import torch

    M, K = X.shape
    _check_rows("X", X, M, K, torch.float32)
    if X.stride(0) % 4:
        raise ValueError("X's row stride must be a multiple of 4 elements")
    for name, t, dt, n in (("Wp", Wp, torch.int8, lib().hq_int8_packed_bytes(K, N)), ("scales", scales, torch.float32, N)):
        if t.device != X.device or t.dtype != dt or not t.is_contiguous() or t.numel() < n:
            raise ValueError(f"{name} must be a contiguous {dt} device tensor of at least {n} elements on X's device")
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=X.device)
    _check_rows("out", out, M, N, torch.float32)
    wp, wb = _ws(workspace)
    check(lib().hq_gemm_w8a8(X.data_ptr(), X.stride(0), Wp.data_ptr(), scales.data_ptr(), out.data_ptr(), out.stride(0),
                             M, K, N, wp, wb, _stream_ptr(stream)))
    return out
