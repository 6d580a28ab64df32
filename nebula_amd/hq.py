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

DTYPE_F16 = 1
DTYPE_BF16 = 2
FORMAT_INT4 = 1
FORMAT_TERNARY2 = 2
MAX_SEGMENTS = 8

# Every symbol include/hq_qgemm.h declares.
EXPORTS = (
    "hq_version", "hq_last_error", "hq_status_string", "hq_linear_words", "hq_packed_words",
    "hq_workspace_bytes", "hq_repack_int4_ref", "hq_repack_int4", "hq_repack_ternary2",
    "hq_unpack_int4", "hq_unpack_ternary2", "hq_repack_int4_device", "hq_repack_ternary2_device",
    "hq_gemm_w4a16", "hq_gemm_w2a16", "hq_gemm_fused", "hq_tq1_0_bytes", "hq_convert_tq1_0",
    "hq_repack_tq1_0_device",
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
    for name in ("hq_repack_int4_ref", "hq_repack_int4", "hq_repack_ternary2", "hq_unpack_int4", "hq_unpack_ternary2"):
        f = getattr(L, name)
        f.restype = i32
        f.argtypes = [vp, vp, u32, u32]
    L.hq_repack_int4_device.restype = i32
    L.hq_repack_int4_device.argtypes = [vp, vp, u32, u32, vp]
    L.hq_repack_ternary2_device.restype = i32
    L.hq_repack_ternary2_device.argtypes = [vp, vp, u32, u32, vp, vp]
    for name in ("hq_gemm_w4a16", "hq_gemm_w2a16"):
        f = getattr(L, name)
        f.restype = i32
        f.argtypes = [vp, i32, i64, vp, vp, vp, i64, u32, u32, u32, u32, vp, sz, vp]
    L.hq_tq1_0_bytes.restype = sz
    L.hq_tq1_0_bytes.argtypes = [u32, u32]
    L.hq_convert_tq1_0.restype = i32
    L.hq_convert_tq1_0.argtypes = [vp, u32, u32, vp, vp]
    L.hq_repack_tq1_0_device.restype = i32
    L.hq_repack_tq1_0_device.argtypes = [vp, u32, u32, vp, vp, vp]
    L.hq_gemm_fused.restype = i32
    L.hq_gemm_fused.argtypes = [vp, i32, i64, i32, ctypes.POINTER(Segment), u32, u32, u32, u32, vp, sz, vp]
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
    """Bytes of the decode fix-up workspace for this shape on the current device (0: none)."""
    b = ctypes.c_size_t(0)
    check(lib().hq_workspace_bytes(fmt, M, K, N, group, ctypes.byref(b)))
    return int(b.value)


def _ws(workspace):
    """(pointer, bytes) of a caller workspace tensor (zero-filled before first use), or (None, 0)."""
    if workspace is None:
        return None, 0
    return workspace.data_ptr(), workspace.numel() * workspace.element_size()


def gemm(fmt: int, X, Wp, scales, N: int, group: int = 128, out=None, stream=None, workspace=None):
    """Y[M, N] = X[M, K] @ dequant(Wp) with fp32 accumulation (Y in X's dtype).

    workspace: optional device tensor of at least workspace_bytes() bytes, zero-filled
    before its first use; by default the library's own per-stream buffer is used."""
    import torch

    M, K = X.shape
    if out is None:
        out = torch.empty((M, N), dtype=X.dtype, device=X.device)
    f = lib().hq_gemm_w4a16 if fmt == FORMAT_INT4 else lib().hq_gemm_w2a16
    wp, wb = _ws(workspace)
    check(f(X.data_ptr(), _dt(X), X.stride(0), Wp.data_ptr(), scales.data_ptr(), out.data_ptr(), out.stride(0),
            M, K, N, group, wp, wb, _stream_ptr(stream)))
    return out


def gemm_fused(fmt: int, X, segments: Sequence[tuple], group: int = 128, outs=None, stream=None, workspace=None):
    """segments: (Wp, scales, N) per projection; returns one output per segment."""
    import torch

    M, K = X.shape
    if outs is None:
        outs = [torch.empty((M, n), dtype=X.dtype, device=X.device) for (_, _, n) in segments]
    arr = (Segment * len(segments))()
    for i, ((wp, sc, n), y) in enumerate(zip(segments, outs)):
        arr[i] = Segment(wp.data_ptr(), sc.data_ptr(), y.data_ptr(), y.stride(0), n)
    wp, wb = _ws(workspace)
    check(lib().hq_gemm_fused(X.data_ptr(), _dt(X), X.stride(0), fmt, arr, len(segments), M, K, group, wp, wb,
                              _stream_ptr(stream)))
    return outs
