"""Writes small synthetic GGUF files for the loader tests, byte by byte in the layout that
hydrogen's parser reads (hydrogen/src/model/tensor_loader.cpp, parse_gguf):

    u32 magic "GGUF", u32 version, u64 tensor_count, u64 kv_count,
    kv_count x (string key, u32 value type, value),
    tensor_count x (string name, u32 n_dims, n_dims x u64 dim, u32 ggml type, u64 offset),
    padding to the alignment (general.alignment, default 32), then the tensor data,
    each tensor at its offset from the start of the data;

strings are u64 length + bytes, arrays u32 element type + u64 count + elements, all
little-endian. Also encodes GGML Q4_K blocks from chosen scales, mins and codes
(the published block_q4_K: fp16 d, fp16 dmin, 12 bytes of 6-bit scales and mins, 128 bytes
of nibbles). Used by tests/test_gguf.py and tests/test_gpu_gguf.py; run as a script it writes
an example file.
"""
from __future__ import annotations

import struct
import sys

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}
BLOCK = {0: (1, 4), 1: (1, 2), 12: (256, 144), 34: (256, 56), 143: (256, 56), 8: (32, 34)}


def _str(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    if t == STRING:
        return _str(v)
    if t == ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def gguf_bytes(kv, tensors, version: int = 3, alignment: int | None = None, raw_header: bytes | None = None) -> bytes:
    """kv: [(key, type, value)]; tensors: [(name, shape, ggml_type, data bytes or None, offset or None)].
    Offsets default to consecutive aligned placement; data None leaves the tensor out of the data."""
    align = alignment if alignment else 32
    out = bytearray(raw_header if raw_header is not None else struct.pack("<IIQQ", 0x46554747, version, len(tensors),
                                                                           len(kv)))
    for key, t, v in kv:
        out += _str(key) + struct.pack("<I", t) + _value(t, v)
    placed, off = [], 0
    for name, shape, gt, data, offset in tensors:
        if offset is None:
            offset = off
        nbytes = len(data) if data is not None else 0
        off = max(off, (offset + nbytes + align - 1) // align * align)
        placed.append((offset, data))
        out += _str(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        out += struct.pack("<IQ", gt, offset)
    start = (len(out) + align - 1) // align * align
    out += b"\0" * (start - len(out))
    end = start + max([o + len(d) for o, d in placed if d is not None] + [0])
    body = bytearray(end - start)
    for o, d in placed:
        if d is not None:
            body[o:o + len(d)] = d
    return bytes(out + body)


def f16_bits(x: float) -> int:
    return int(np.array([x], dtype=np.float16).view(np.uint16)[0])


def q4_k_block(d: float, dmin: float, sc, m, q) -> bytes:
    """One Q4_K block from sub-block scales sc[8], mins m[8] (6-bit) and codes q[256] (4-bit)."""
    sc, m, q = [int(x) for x in sc], [int(x) for x in m], np.asarray(q, dtype=np.uint8)
    s = [0] * 12
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    qs = bytearray(128)
    for c in range(4):
        for l in range(32):
            qs[32 * c + l] = int(q[64 * c + l]) | (int(q[64 * c + 32 + l]) << 4)
    return struct.pack("<HH", f16_bits(d), f16_bits(dmin)) + bytes(s) + bytes(qs)


def q4_k_expected(d: float, dmin: float, sc, m, q) -> np.ndarray:
    """The block's 256 weights, (d * sc) * q - dmin * m in float32 with separate roundings."""
    d32, m32 = np.float32(np.float16(d)), np.float32(np.float16(dmin))
    j = np.arange(256) // 32
    d1 = d32 * np.asarray(sc, dtype=np.float32)[j]
    m1 = m32 * np.asarray(m, dtype=np.float32)[j]
    return d1 * np.asarray(q, dtype=np.float32) - m1


def random_q4_k(rng, K: int, N: int):
    """N rows of K/256 random Q4_K blocks (bytes) and their float32 weights [K, N]."""
    nb = K // 256
    raw, W = bytearray(), np.empty((K, N), dtype=np.float32)
    for n in range(N):
        for b in range(nb):
            d, dmin = float(rng.uniform(1e-4, 3e-3)), float(rng.uniform(1e-4, 3e-3))
            sc, mn, q = rng.integers(0, 64, 8), rng.integers(0, 64, 8), rng.integers(0, 16, 256)
            raw += q4_k_block(d, dmin, sc, mn, q)
            W[256 * b:256 * (b + 1), n] = q4_k_expected(d, dmin, sc, mn, q)
    return np.frombuffer(bytes(raw), dtype=np.uint8).copy(), W


def example() -> bytes:
    rng = np.random.default_rng(0)
    tq = rng.integers(0, 256, 4 * 2 * 56, dtype=np.uint8).tobytes()
    q4, _ = random_q4_k(rng, 256, 2)
    kv = [("general.architecture", STRING, "qwen35"), ("qwen35.block_count", U32, 1),
          ("general.alignment", U32, 32), ("tokenizer.ggml.tokens", ARRAY, (STRING, ["a", "bc"]))]
    tensors = [("blk.0.attn_q.weight", [512, 4], 143, tq, None), ("blk.0.ffn_up.weight", [256, 2], 12, q4.tobytes(), None)]
    return gguf_bytes(kv, tensors)


if __name__ == "__main__":
    path = sys.argv[1] if len(sys.argv) > 1 else "example.gguf"
    with open(path, "wb") as f:
        f.write(example())
    print(path)
