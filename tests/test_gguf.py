"""CPU tests of the GGUF container loader (hq_gguf_*), against files written byte by byte by
tests/golden/make_gguf.py in the layout hydrogen's parser reads
(hydrogen/src/model/tensor_loader.cpp), and of the GGML Q4_K import against the oracle's
restatement of the published Q4_K dequantisation.

The reference parser's rules are checked one by one: magic, versions 2..3 only, typed
metadata of every value type (nested arrays, string arrays), general.alignment (default 32, 0
read as 32), tensor data at the aligned end of the header, sizes from the type's block traits,
a null data pointer past the end of the data, at most 4 dimensions, the last of a repeated
tensor name winning. Every prefix of a file parses or fails with HQ_ERR_FORMAT.
"""
import struct
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from nebula_amd import gguf as G
from nebula_amd import hq

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_gguf as MG  # noqa: E402

RNG = np.random.default_rng(77)


def sample_file():
    tq = RNG.integers(0, 256, 3 * 2 * 56, dtype=np.uint8).tobytes()  # [512, 3] TQ1_0
    f32 = np.arange(7, dtype=np.float32).tobytes()
    q4, W = MG.random_q4_k(RNG, 512, 2)
    kv = [("general.architecture", MG.STRING, "qwen35"), ("qwen35.block_count", MG.U32, 64),
          ("qwen35.embedding_length", MG.U64, 5120), ("i8", MG.I8, -5), ("u16", MG.U16, 65535),
          ("i16", MG.I16, -300), ("i32", MG.I32, -70000), ("i64", MG.I64, -(2**40)), ("u8", MG.U8, 200),
          ("eps", MG.F32, 1e-6), ("rope", MG.F64, 1e6), ("flag", MG.BOOL, 1),
          ("tokenizer.ggml.tokens", MG.ARRAY, (MG.STRING, ["<s>", "hello", ""])),
          ("nested", MG.ARRAY, (MG.ARRAY, [(MG.U32, [1, 2, 3]), (MG.STRING, ["x"])]))]
    tensors = [("blk.3.attn_q.weight", [512, 3], 143, tq, None), ("output_norm.weight", [7], 0, f32, None),
               ("blk.0.ffn_up.weight", [512, 2], 12, q4.tobytes(), None),
               ("blk.3.attn_k.weight", [256, 2], 34, tq[:2 * 56], None)]
    return MG.gguf_bytes(kv, tensors), tq, f32, q4, W


def test_header_metadata_and_directory(tmp_path):
    data, tq, f32, q4, _ = sample_file()
    p = tmp_path / "m.gguf"
    p.write_bytes(data)
    with G.GGUF(path=str(p)) as g:
        h = g.header
        assert h["version"] == 3 and h["tensor_count"] == 4 and h["kv_count"] == 14 and h["alignment"] == 32
        assert h["tensor_data_offset"] % 32 == 0 and h["tensor_data_offset"] - h["header_bytes"] < 32
        assert h["file_bytes"] == len(data)
        assert g.get_string("general.architecture") == "qwen35"
        assert g.get_int("qwen35.block_count") == 64 and g.get_int("qwen35.embedding_length") == 5120
        assert (g.get_int("i8"), g.get_int("u16"), g.get_int("i16"), g.get_int("i32"), g.get_int("i64"),
                g.get_int("u8"), g.get_int("flag")) == (-5, 65535, -300, -70000, -(2**40), 200, 1)
        assert g.get_float("eps") == pytest.approx(1e-6, rel=1e-7) and g.get_float("rope") == 1e6
        assert g.get_array("tokenizer.ggml.tokens") == (MG.STRING, 3)
        assert g.get_array("nested") == (MG.ARRAY, 2)
        assert g.get_int("missing", 9) == 9
        with pytest.raises(hq.HQError) as ei:
            g.get_int("general.architecture")
        assert ei.value.status == hq.HQ_ERR_INVALID_ARG
        ts = {t["name"]: t for t in g.tensors()}
        assert ts["blk.3.attn_q.weight"]["shape"] == [512, 3] and ts["blk.3.attn_q.weight"]["size_bytes"] == 3 * 2 * 56
        assert ts["output_norm.weight"]["size_bytes"] == 28 and ts["blk.0.ffn_up.weight"]["size_bytes"] == 2 * 2 * 144
        for t in ts.values():
            assert t["absolute_offset"] == h["tensor_data_offset"] + t["offset"] and t["offset"] % 32 == 0
        assert g.tensor_bytes("blk.3.attn_q.weight").tobytes() == tq
        assert g.tensor_bytes("output_norm.weight").tobytes() == f32
        assert g.tensor_bytes("blk.0.ffn_up.weight").tobytes() == q4.tobytes()
        assert g.find("nope") is None
    # The same bytes parsed from memory.
    with G.GGUF(data=data) as g:
        assert g.header["tensor_count"] == 4 and g.find("output_norm.weight")["size_bytes"] == 28


@pytest.mark.parametrize("align,expect", [(None, 32), (0, 32), (64, 64), (256, 256)])
def test_alignment_rule(align, expect):
    kv = [] if align is None else [("general.alignment", MG.U32, align)]
    data = MG.gguf_bytes(kv, [("t", [4], 0, b"\1" * 16, None), ("u", [3], 0, b"\2" * 12, None)], alignment=expect)
    with G.GGUF(data=data) as g:
        h = g.header
        assert h["alignment"] == expect and h["tensor_data_offset"] % expect == 0
        assert g.tensor_bytes("u").tobytes() == b"\2" * 12


def status_of(data: bytes) -> int:
    try:
        G.GGUF(data=data).close()
        return hq.HQ_OK
    except hq.HQError as e:
        return e.status


def test_rejects_what_the_reference_rejects():
    good, *_ = sample_file()
    assert status_of(good) == hq.HQ_OK
    assert status_of(b"GGUX" + good[4:]) == hq.HQ_ERR_FORMAT  # magic
    for v in (1, 4):
        assert status_of(good[:4] + struct.pack("<I", v) + good[8:]) == hq.HQ_ERR_FORMAT  # version
    assert status_of(good[:4] + struct.pack("<I", 2) + good[8:]) == hq.HQ_OK  # version 2 is read
    assert status_of(good[:20]) == hq.HQ_ERR_FORMAT  # shorter than a header
    five = MG.gguf_bytes([], [("t", [1, 1, 1, 1, 2], 0, b"\0" * 8, None)])
    assert status_of(five) == hq.HQ_ERR_FORMAT  # more than 4 dimensions
    bad_type = MG.gguf_bytes([("k", MG.U32, 1)], [])
    bad_type = bad_type.replace(struct.pack("<Q", 1) + b"k" + struct.pack("<I", MG.U32),
                                struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13))
    assert status_of(bad_type) == hq.HQ_ERR_FORMAT  # unknown value type


def test_every_prefix_parses_or_fails_cleanly():
    good, *_ = sample_file()
    h_end = G.GGUF(data=good).header["header_bytes"]
    for n in range(0, h_end):
        assert status_of(good[:n]) == hq.HQ_ERR_FORMAT, n
    # Past the directory the parse succeeds; tensors beyond the data have no data pointer.
    with G.GGUF(data=good[:len(good) - 1]) as g:
        last = max(g.tensors(), key=lambda t: t["absolute_offset"] + t["size_bytes"])
        assert not last["in_file"]
        with pytest.raises(ValueError):
            g.tensor_bytes(last["name"])


def test_repeated_name_last_wins_and_unknown_types():
    data = MG.gguf_bytes([], [("w", [4], 0, b"\1" * 16, None), ("w", [8], 1, b"\2" * 16, None),
                              ("odd", [5], 200, b"\3" * 5, None)])
    with G.GGUF(data=data) as g:
        assert g.find("w")["shape"] == [8] and g.find("w")["type"] == 1
        assert g.find("odd")["size_bytes"] == 5  # unlisted type: one byte per element


def test_tq1_0_tensor_converts_like_its_blocks():
    data, tq, *_ = sample_file()
    with G.GGUF(data=data) as g:
        raw = g.tensor_bytes("blk.3.attn_q.weight")
    codes, scales = hq.convert_tq1_0(raw, 512, 3)
    ref_codes, ref_scales = hq.convert_tq1_0(np.frombuffer(tq, dtype=np.uint8), 512, 3)
    assert np.array_equal(codes, ref_codes) and np.array_equal(scales, ref_scales)
    blocks = np.frombuffer(tq, dtype=np.uint8).reshape(3, 2, 56)
    for n in range(3):
        for b in range(2):
            assert np.array_equal((codes.reshape(32, 3)[16 * b:16 * (b + 1), n][:, None] >>
                                   (2 * np.arange(16, dtype=np.uint32))[None, :] & 3).ravel(), O.tq1_0_codes(blocks[n, b]))


# ---------------------------------------------------------------- GGML Q4_K
def test_oracle_q4_k_matches_the_block_encoder():
    # Every 6-bit scale and min value in both halves of the scale bytes, every code.
    for trial in range(8):
        sc = RNG.integers(0, 64, 8)
        m = RNG.integers(0, 64, 8)
        sc[trial % 8], m[(trial + 3) % 8] = 63, 63
        q = RNG.integers(0, 16, 256)
        d, dmin = float(RNG.uniform(1e-4, 2e-2)), float(RNG.uniform(1e-4, 2e-2))
        blk = np.frombuffer(MG.q4_k_block(d, dmin, sc, m, q), dtype=np.uint8)
        got = O.dequant_q4_k(blk, 256, 1)[:, 0]
        assert np.array_equal(got.view(np.uint32), MG.q4_k_expected(d, dmin, sc, m, q).view(np.uint32))
    # A wrong nibble order (high nibble first) would not match.
    q = np.arange(256) % 16
    blk = np.frombuffer(MG.q4_k_block(1e-2, 0.0, [1] * 8, [0] * 8, q), dtype=np.uint8)
    assert not np.array_equal(O.dequant_q4_k(blk, 256, 1)[:, 0], np.float32(np.float16(1e-2)) * q[::-1])


def test_oracle_q4_k_known_answer_block():
    # One block written byte by byte (no encoder): d = 1.0, dmin = 0.5 (fp16), scale bytes whose
    # top two bits feed sub-blocks 4..7. Sub-block scales and mins worked out by hand from GGML's
    # published layout (get_scale_min_k4: j < 4 from bytes j and j + 4, low six bits; j >= 4 the
    # low / high nibble of byte j + 4 below the top two bits of byte j - 4 / j):
    #   scales 1, 2, 3, 4, 26, 12, 14, 48 and mins 5, 6, 7, 8, 9, 11, 29, 47.
    # Codes: byte l of qs holds l % 16 in its low nibble and 15 - l % 16 in its high nibble; the
    # 64 weights of chunk c are the 32 low nibbles of bytes 32c.. (sub-block 2c), then their
    # 32 high nibbles (sub-block 2c + 1). Every weight sc * q - 0.5 * m is exact in float32.
    scale_bytes = [0x41, 0x02, 0x03, 0xC4, 0x05, 0x06, 0x47, 0x88, 0x9A, 0xBC, 0xDE, 0xF0]
    qs = [(l % 16) | ((15 - l % 16) << 4) for l in range(128)]
    blk = np.frombuffer(bytes([0x00, 0x3C, 0x00, 0x38] + scale_bytes + qs), dtype=np.uint8)
    assert blk.size == 144
    sc = [1, 2, 3, 4, 26, 12, 14, 48]
    mn = [5, 6, 7, 8, 9, 11, 29, 47]
    want = np.empty(256, dtype=np.float32)
    for i in range(256):
        c, l, hi = i // 64, i % 32, (i % 64) >= 32
        q = 15 - l % 16 if hi else l % 16
        j = 2 * c + (1 if hi else 0)
        want[i] = sc[j] * q - 0.5 * mn[j]
    got = O.dequant_q4_k(blk, 256, 1)[:, 0]
    assert np.array_equal(got, want), np.flatnonzero(got != want)[:8]
    # Spot values: weight 0 is 1 * 0 - 2.5, weight 32 is 2 * 15 - 3, weight 255 is 48 * 0 - 23.5.
    assert (got[0], got[32], got[255]) == (-2.5, 27.0, -23.5)


@pytest.mark.parametrize("K,N", [(256, 1), (512, 3), (1024, 40)])
def test_convert_q4_k_is_the_published_weight(K, N):
    raw, W = MG.random_q4_k(RNG, K, N)
    codes, scales, bias = G.convert_q4_k(raw, K, N)
    # The import, read back with the reference's q * s + b (groups of 32), is the Q4_K weight with
    # its scale d * sc rounded to fp16 (the only loss; the bias -dmin * m is exact in fp32).
    mine = O.dequant_int4_bias(codes, scales, bias, K, N, 32)
    ref = O.dequant_q4_k(raw, K, N)
    assert np.array_equal(ref.view(np.uint32), W.view(np.uint32))
    qv = np.empty((K, N), dtype=np.float32)
    for k in range(K):
        qv[k] = (codes.reshape(K // 8, N)[k // 8] >> (4 * (k % 8))) & 15
    s = np.repeat(O.to_f32(scales, O.F16), 32, axis=0)
    b = np.repeat(bias, 32, axis=0)
    assert np.array_equal(mine.view(np.uint32), (qv * s + b).view(np.uint32))
    assert np.all(np.abs(mine.astype(np.float64) - ref) <= 2.0**-11 * (qv * np.abs(s)) + 1e-12)
    # Through an open file as well.
    data = MG.gguf_bytes([], [("blk.0.ffn_up.weight", [K, N], 12, raw.tobytes(), None)])
    with G.GGUF(data=data) as g:
        c2, s2, b2, k2, n2 = g.convert_q4_k("blk.0.ffn_up.weight")
    assert (k2, n2) == (K, N) and np.array_equal(c2, codes) and np.array_equal(s2, scales) and np.array_equal(b2, bias)


def test_typed_loads_check_type_and_shape():
    data, *_ = sample_file()
    with G.GGUF(data=data) as g:
        with pytest.raises(hq.HQError) as ei:
            g.convert_q4_k("blk.3.attn_q.weight")  # a TQ1_0 tensor
        assert ei.value.status == hq.HQ_ERR_UNSUPPORTED
        with pytest.raises(hq.HQError) as ei:
            g.convert_q4_k("output_norm.weight")
        assert ei.value.status in (hq.HQ_ERR_UNSUPPORTED, hq.HQ_ERR_SHAPE)
        with pytest.raises(KeyError):
            g.convert_q4_k("nope")


def test_open_missing_file_is_an_io_error(tmp_path):
    with pytest.raises(hq.HQError) as ei:
        G.GGUF(path=str(tmp_path / "none.gguf"))
    assert ei.value.status == hq.HQ_ERR_IO
