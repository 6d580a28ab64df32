"""GGUF container access through the library's C ABI (hq_gguf_*, include/hq_qgemm.h).

Replaces, for the weights of this path, hydrogen's ModelLoader / parse_gguf
(hydrogen/include/tensor_loader.hpp:14-53, hydrogen/include/gguf_parser.hpp:33-145,
hydrogen/src/model/tensor_loader.cpp): the file is memory-mapped and parsed by the library;
TQ1_0 projections are repacked on the device at load (hq_gguf_load_tq1_0) and Q4_K ones
converted on the host into int4 codes, fp16 scales and fp32 biases with groups of 32
(hq_gguf_convert_q4_k). `load_layer` builds a decoder layer's projections from the tensor
names the reference decoder looks up (hydrogen/src/model/native_decoder.cu:874-913).
"""
from __future__ import annotations

import ctypes
from typing import Dict, Optional

import numpy as np

from . import hq

GGML_F32, GGML_F16, GGML_Q4_K, GGML_TQ1_0, GGML_TQ1_0_PRISM = 0, 1, 12, 34, 143


class HeaderInfo(ctypes.Structure):
    _fields_ = [("version", ctypes.c_uint32), ("tensor_count", ctypes.c_uint64), ("kv_count", ctypes.c_uint64),
                ("alignment", ctypes.c_uint64), ("header_bytes", ctypes.c_uint64),
                ("tensor_data_offset", ctypes.c_uint64), ("total_tensor_bytes", ctypes.c_uint64),
                ("file_bytes", ctypes.c_uint64)]


class TensorInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("n_dims", ctypes.c_uint32), ("shape", ctypes.c_uint64 * 4),
                ("type", ctypes.c_uint32), ("offset", ctypes.c_uint64), ("absolute_offset", ctypes.c_uint64),
                ("size_bytes", ctypes.c_uint64), ("data", ctypes.c_void_p)]

    def as_dict(self) -> dict:
        return {"name": self.name.decode(), "shape": list(self.shape[:self.n_dims]), "type": int(self.type),
                "offset": int(self.offset), "absolute_offset": int(self.absolute_offset),
                "size_bytes": int(self.size_bytes), "in_file": bool(self.data)}


_bound = False


def _lib():
    global _bound
    L = hq.lib()
    if _bound:
        return L
    vp, u32, u64, sz, i32, cp = (ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_size_t, ctypes.c_int,
                                 ctypes.c_char_p)
    L.hq_gguf_open.restype = i32
    L.hq_gguf_open.argtypes = [cp, ctypes.POINTER(vp)]
    L.hq_gguf_parse.restype = i32
    L.hq_gguf_parse.argtypes = [vp, sz, ctypes.POINTER(vp)]
    L.hq_gguf_close.restype = None
    L.hq_gguf_close.argtypes = [vp]
    L.hq_gguf_header.restype = i32
    L.hq_gguf_header.argtypes = [vp, ctypes.POINTER(HeaderInfo)]
    L.hq_gguf_tensor_at.restype = i32
    L.hq_gguf_tensor_at.argtypes = [vp, u64, ctypes.POINTER(TensorInfo)]
    L.hq_gguf_find_tensor.restype = i32
    L.hq_gguf_find_tensor.argtypes = [vp, cp, ctypes.POINTER(TensorInfo)]
    L.hq_gguf_get_int.restype = i32
    L.hq_gguf_get_int.argtypes = [vp, cp, ctypes.POINTER(ctypes.c_int64)]
    L.hq_gguf_get_float.restype = i32
    L.hq_gguf_get_float.argtypes = [vp, cp, ctypes.POINTER(ctypes.c_double)]
    L.hq_gguf_get_string.restype = i32
    L.hq_gguf_get_string.argtypes = [vp, cp, ctypes.c_char_p, sz, ctypes.POINTER(sz)]
    L.hq_gguf_get_array.restype = i32
    L.hq_gguf_get_array.argtypes = [vp, cp, ctypes.POINTER(u32), ctypes.POINTER(u64)]
    L.hq_gguf_load_tq1_0.restype = i32
    L.hq_gguf_load_tq1_0.argtypes = [vp, cp, vp, sz, vp, vp, ctypes.POINTER(u32), ctypes.POINTER(u32), vp]
    L.hq_convert_q4_k.restype = i32
    L.hq_convert_q4_k.argtypes = [vp, u32, u32, vp, vp, vp]
    L.hq_gguf_convert_q4_k.restype = i32
    L.hq_gguf_convert_q4_k.argtypes = [vp, cp, vp, vp, vp, ctypes.POINTER(u32), ctypes.POINTER(u32)]
    _bound = True
    return L


class GGUF:
    """An open GGUF file (memory-mapped by the library) or a parsed byte buffer."""

    def __init__(self, path: Optional[str] = None, data: Optional[bytes] = None):
        L = _lib()
        h = ctypes.c_void_p()
        self._keep = None
        if path is not None:
            hq.check(L.hq_gguf_open(str(path).encode(), ctypes.byref(h)))
        elif data is not None:
            self._keep = ctypes.create_string_buffer(bytes(data), len(data))
            hq.check(L.hq_gguf_parse(self._keep, len(data), ctypes.byref(h)))
        else:
            raise ValueError("need a path or data")
        self._h = h

    def close(self) -> None:
        if self._h:
            _lib().hq_gguf_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 - interpreter shutdown
            pass

    @property
    def header(self) -> dict:
        info = HeaderInfo()
        hq.check(_lib().hq_gguf_header(self._h, ctypes.byref(info)))
        return {f: int(getattr(info, f)) for f, _ in HeaderInfo._fields_}

    def tensors(self):
        n = self.header["tensor_count"]
        out = []
        for i in range(n):
            t = TensorInfo()
            hq.check(_lib().hq_gguf_tensor_at(self._h, i, ctypes.byref(t)))
            out.append(t.as_dict())
        return out

    def find(self, name: str) -> Optional[dict]:
        t = TensorInfo()
        st = _lib().hq_gguf_find_tensor(self._h, name.encode(), ctypes.byref(t))
        if st == hq.HQ_ERR_NOT_FOUND:
            return None
        hq.check(st)
        return t.as_dict()

    def tensor_bytes(self, name: str) -> np.ndarray:
        """The tensor's bytes (a copy out of the mapping)."""
        t = TensorInfo()
        hq.check(_lib().hq_gguf_find_tensor(self._h, name.encode(), ctypes.byref(t)))
        if not t.data:
            raise ValueError(f"tensor {name} extends past the end of the data")
        return np.ctypeslib.as_array((ctypes.c_uint8 * t.size_bytes).from_address(t.data)).copy()

    def get_int(self, key: str, default=None):
        v = ctypes.c_int64()
        st = _lib().hq_gguf_get_int(self._h, key.encode(), ctypes.byref(v))
        if st == hq.HQ_ERR_NOT_FOUND and default is not None:
            return default
        hq.check(st)
        return int(v.value)

    def get_float(self, key: str, default=None):
        v = ctypes.c_double()
        st = _lib().hq_gguf_get_float(self._h, key.encode(), ctypes.byref(v))
        if st == hq.HQ_ERR_NOT_FOUND and default is not None:
            return default
        hq.check(st)
        return float(v.value)

    def get_string(self, key: str, default=None):
        n = ctypes.c_size_t()
        L = _lib()
        st = L.hq_gguf_get_string(self._h, key.encode(), None, 0, ctypes.byref(n))
        if st == hq.HQ_ERR_NOT_FOUND and default is not None:
            return default
        hq.check(st)
        buf = ctypes.create_string_buffer(n.value + 1)
        hq.check(L.hq_gguf_get_string(self._h, key.encode(), buf, len(buf), None))
        return buf.raw[:n.value].decode("utf-8", errors="replace")

    def get_array(self, key: str):
        """(element type, count) of an array-valued key."""
        t, n = ctypes.c_uint32(), ctypes.c_uint64()
        hq.check(_lib().hq_gguf_get_array(self._h, key.encode(), ctypes.byref(t), ctypes.byref(n)))
        return int(t.value), int(n.value)

    def load_tq1_0(self, name: str, stream=None):
        """A TQ1_0 projection onto the device: (packed ternary tiles, fp16 scales [K/256, N], K, N)."""
        import torch

        info = self.find(name)
        if info is None:
            raise KeyError(name)
        if len(info["shape"]) != 2:
            raise ValueError(f"{name} is not a matrix: shape {info['shape']}")
        K, N = info["shape"]
        staging = torch.empty(info["size_bytes"], dtype=torch.uint8, device="cuda")
        packed = torch.empty(hq.packed_words(hq.FORMAT_TERNARY2, K, N), dtype=torch.int32, device="cuda")
        scales = torch.empty((K // 256, N), dtype=torch.float16, device="cuda")
        k, n = ctypes.c_uint32(), ctypes.c_uint32()
        s = stream if stream is not None else torch.cuda.current_stream()
        hq.check(_lib().hq_gguf_load_tq1_0(self._h, name.encode(), staging.data_ptr(), staging.numel(),
                                           packed.data_ptr(), scales.data_ptr(), ctypes.byref(k), ctypes.byref(n),
                                           s.cuda_stream))
        s.synchronize()  # the copy reads the mapping; the staging buffer may go after this
        return packed, scales, int(k.value), int(n.value)

    def convert_q4_k(self, name: str):
        """A Q4_K weight as (int4 linear codes [K/8 * N], fp16 scale bits [K/32, N], fp32 biases
        [K/32, N], K, N): the inputs of hq.repack and hq.gemm(..., bias=..., group=32)."""
        info = self.find(name)
        if info is None:
            raise KeyError(name)
        k, n = ctypes.c_uint32(), ctypes.c_uint32()
        if len(info["shape"]) != 2 or info["type"] != GGML_Q4_K:  # the library reports what is wrong
            hq.check(_lib().hq_gguf_convert_q4_k(self._h, name.encode(), None, None, None, ctypes.byref(k),
                                                 ctypes.byref(n)))
        K, N = info["shape"]
        codes = np.empty((K // 8) * N, dtype=np.uint32)
        scales = np.empty((K // 32, N), dtype=np.uint16)
        bias = np.empty((K // 32, N), dtype=np.float32)
        hq.check(_lib().hq_gguf_convert_q4_k(self._h, name.encode(), codes.ctypes.data, scales.ctypes.data,
                                             bias.ctypes.data, ctypes.byref(k), ctypes.byref(n)))
        return codes, scales, bias, int(k.value), int(n.value)


def convert_q4_k(blocks: np.ndarray, K: int, N: int):
    """GGML Q4_K blocks (N rows of K/256 blocks of 144 bytes) -> (codes, fp16 scale bits, fp32 biases)."""
    src = np.ascontiguousarray(blocks, dtype=np.uint8)
    if src.size != N * (K // 256) * 144:
        raise ValueError(f"Q4_K tensor has {src.size} bytes, expected {N * (K // 256) * 144}")
    codes = np.empty((K // 8) * N, dtype=np.uint32)
    scales = np.empty((K // 32, N), dtype=np.uint16)
    bias = np.empty((K // 32, N), dtype=np.float32)
    hq.check(_lib().hq_convert_q4_k(src.ctypes.data, K, N, codes.ctypes.data, scales.ctypes.data, bias.ctypes.data))
    return codes, scales, bias


# GGUF tensor names of a decoder layer's projections (native_decoder.cu:876-913) -> the names
# nebula_amd.decoder uses.
LAYER_TENSORS = {
    "attention": {"attn_q": "attn_q", "attn_k": "attn_k", "attn_v": "attn_v", "attn_output": "attn_output"},
    "ssm": {"ssm_gate": "attn_gate", "ssm_qkv": "attn_qkv", "ssm_out": "ssm_out"},
    "ffn": {"ffn_gate": "ffn_gate", "ffn_up": "ffn_up", "ffn_down": "ffn_down"},
}


def layer_kind(layer: int) -> str:
    """Every fourth layer is an attention layer, the others SSM layers (native_decoder.cu:890)."""
    return "attention" if layer % 4 == 3 else "ssm"


def load_layer(g: GGUF, layer: int, stream=None):
    """The TQ1_0 projections of decoder layer `layer` as a decoder.LayerProjections."""
    from . import decoder

    kind = layer_kind(layer)
    w: Dict[str, decoder.TernaryProjection] = {}
    for ours, theirs in {**LAYER_TENSORS[kind], **LAYER_TENSORS["ffn"]}.items():
        Wp, S, K, N = g.load_tq1_0(f"blk.{layer}.{theirs}.weight", stream=stream)
        w[ours] = decoder.TernaryProjection(K, N, Wp, S)
    return decoder.LayerProjections(kind, w)
