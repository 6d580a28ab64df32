"""GPU tests of weights imported from GGUF files (tests/golden/make_gguf.py writes them):

* TQ1_0 tensors (types 143 and 34) loaded onto the device by hq_gguf_load_tq1_0 equal the host
  conversion + host repack of the same blocks, and GEMMs on them match the oracle's restatement
  of kernel_gemv_tq1_0 (hydrogen/src/model/native_decoder.cu:155-206);
* Q4_K tensors converted by hq_gguf_convert_q4_k run as int4 weights with a bias and groups of
  32 and match the oracle's X @ dequant_q4_k (the published dequantisation) within the fp16
  rounding of the scale d * sc (2^-11 relative), the only loss of the import;
* a decoder attention layer at the 27B shapes is loaded by name (native_decoder.cu:874-913)
  and its fused projections match the oracle on sampled rows.
"""
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from gpu_util import to_dev_u16, to_dev_u32, to_host_f32
from nebula_amd import decoder as D
from nebula_amd import gguf as G
from nebula_amd import hq

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_gguf as MG  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("gtype", [143, 34])
@pytest.mark.parametrize("K,N,M", [(512, 40, 1), (1024, 300, 16), (2048, 1000, 200)])
def test_tq1_0_load_and_gemm(cuda, tmp_path, gtype, K, N, M):
    blocks = O.gen_tq1_0(K + N + gtype, N, K, nonfinite_every=53)
    path = tmp_path / "t.gguf"
    path.write_bytes(MG.gguf_bytes([("general.architecture", MG.STRING, "qwen35")],
                                   [("blk.3.attn_q.weight", [K, N], gtype, blocks.tobytes(), None)]))
    with G.GGUF(path=str(path)) as g:
        Wp, S, k, n = g.load_tq1_0("blk.3.attn_q.weight")
    assert (k, n) == (K, N)
    codes, scales = hq.convert_tq1_0(blocks.reshape(-1), K, N)
    assert np.array_equal(Wp.cpu().numpy().view(np.uint32), hq.repack(hq.FORMAT_TERNARY2, codes, K, N))
    assert np.array_equal(S.cpu().numpy().view(np.uint16), scales)
    X = O.gen_normal(M, 1, M * K, 1.0, False, O.F16).reshape(M, K)
    y = hq.gemm(hq.FORMAT_TERNARY2, to_dev_u16(X, O.F16), Wp, S, N, 256)
    ref = O.gemv_tq1_0(O.to_f32(X, O.F16), blocks, N, threads=16)
    assert O.normwise_error(to_host_f32(y), ref) <= 2e-3


@pytest.mark.parametrize("xdt", [O.F16, O.BF16])
@pytest.mark.parametrize("K,N,M", [(512, 64, 1), (1024, 200, 8), (2048, 520, 64), (1024, 300, 200)])
def test_q4_k_import_and_gemm(cuda, xdt, K, N, M):
    import torch

    raw, W = MG.random_q4_k(np.random.default_rng(K + N + M), K, N)
    data = MG.gguf_bytes([], [("blk.0.ffn_up.weight", [K, N], 12, raw.tobytes(), None)])
    with G.GGUF(data=data) as g:
        codes, scales, bias, k, n = g.convert_q4_k("blk.0.ffn_up.weight")
    Wp = to_dev_u32(hq.repack(hq.FORMAT_INT4, codes, K, N))
    X = O.gen_normal(M + 3, 1, M * K, 1.0, False, xdt).reshape(M, K)
    y = hq.gemm(hq.FORMAT_INT4, to_dev_u16(X, xdt), Wp, to_dev_u16(scales), N, 32,
                bias=torch.from_numpy(bias).cuda())
    Xf = O.to_f32(X, xdt)
    ref = O.gemm_f32(Xf, O.dequant_q4_k(raw, K, N), 16)
    yy = to_host_f32(y)
    err = O.normwise_error(yy, ref)
    assert err <= (2e-3 if xdt == O.F16 else 8e-3), err
    # Per element: the scale's fp16 rounding (2^-11 of q d sc) plus the kernels' own bound.
    qd = np.abs(O.dequant_int4_bias(codes, scales, np.zeros_like(bias), K, N, 32)).astype(np.float64)
    mag = np.abs(Xf).astype(np.float64) @ (np.abs(W).astype(np.float64) + qd)
    rel = 2.0**-10 if xdt == O.F16 else 2.0**-7
    excess = np.abs(yy - ref) - (rel * mag + np.abs(ref) * rel + 2.0**-24)
    assert excess.max() <= 0, excess.max()


def test_decoder_layer_from_gguf(cuda, tmp_path):
    # One attention layer (index 3) and its FFN at the 27B shapes, as TQ1_0 tensors.
    import torch

    layer = 3
    names = {**G.LAYER_TENSORS["attention"], **G.LAYER_TENSORS["ffn"]}
    tensors, blocks = [], {}
    for i, (ours, theirs) in enumerate(names.items()):
        K, N = D.SHAPES[ours]
        blocks[ours] = O.gen_tq1_0(8000 + i, N, K)
        tensors.append((f"blk.{layer}.{theirs}.weight", [K, N], 143, blocks[ours].tobytes(), None))
    path = tmp_path / "layer.gguf"
    path.write_bytes(MG.gguf_bytes([("general.architecture", MG.STRING, "qwen35"),
                                    ("qwen35.block_count", MG.U32, 4)], tensors))
    with G.GGUF(path=str(path)) as g:
        assert G.layer_kind(layer) == "attention" and G.layer_kind(0) == "ssm"
        L = G.load_layer(g, layer)
    M = 4
    X = O.gen_normal(9, 1, M * D.EMBEDDING, 1.0, False, O.F16).reshape(M, D.EMBEDDING)
    outs = L.mixer_in(to_dev_u16(X, O.F16))
    torch.cuda.synchronize()
    for n, y in zip(("attn_q", "attn_k", "attn_v"), outs):
        ref = O.gemv_tq1_0(O.to_f32(X, O.F16), blocks[n], D.SHAPES[n][1], threads=16)
        assert O.normwise_error(to_host_f32(y), ref) <= 2e-3, n
    gate, up = L.ffn_in(to_dev_u16(X, O.F16))
    for n, y in (("ffn_gate", gate), ("ffn_up", up)):
        ref = O.gemv_tq1_0(O.to_f32(X, O.F16), blocks[n], D.FFN, threads=16)
        assert O.normwise_error(to_host_f32(y), ref) <= 2e-3, n
