"""GPU tests of the GGUF TQ1_0 import (the reference's BlockTQ1_0 weights,
hydrogen/src/model/native_decoder.cu:31-36), called through the C ABI:

* the device import writes the same words as the host conversion followed by the host
  repack (bit-exact: integer work), and the same scales;
* a GEMM on imported weights matches the oracle's restatement of kernel_gemv_tq1_0
  (native_decoder.cu:155-206) on the same blocks, blocks with a non-finite d included,
  within the normwise 1e-2 bar (fp32 accumulation on both sides; outputs fp16).
"""
import numpy as np
import pytest

import oracle as O
from gpu_util import assert_parity, to_dev_u16, to_host_f32
from nebula_amd import hq

pytestmark = pytest.mark.gpu


def dev_blocks(blocks):
    import torch

    return torch.from_numpy(np.ascontiguousarray(blocks).reshape(-1)).cuda()


@pytest.mark.parametrize("K,N", [(256, 1), (512, 17), (1280, 40), (5120, 1000)])
def test_device_import_matches_host(cuda, K, N):
    import torch

    blocks = O.gen_tq1_0(K * 3 + N, N, K, nonfinite_every=5)
    codes, scales = hq.convert_tq1_0(blocks, K, N)
    packed_host = hq.repack(hq.FORMAT_TERNARY2, codes, K, N)
    Wp, S = hq.repack_tq1_0_device(dev_blocks(blocks), K, N)
    torch.cuda.synchronize()
    assert np.array_equal(Wp.cpu().numpy().view(np.uint32), packed_host)
    assert np.array_equal(S.cpu().numpy().view(np.uint16), scales)


@pytest.mark.parametrize("M,K,N", [(1, 5120, 1024), (8, 5120, 1024), (16, 2048, 3000), (64, 2048, 1536),
                                   (100, 1024, 2048), (300, 2048, 1536), (600, 1024, 4096)])
def test_gemm_on_imported_weights_matches_gemv(cuda, M, K, N):
    import torch

    blocks = O.gen_tq1_0(M + K + N, N, K, nonfinite_every=9)
    Wp, S = hq.repack_tq1_0_device(dev_blocks(blocks), K, N)
    Xb = O.gen_normal(M, 1, M * K, 1.0, False, O.F16).reshape(M, K)
    Y = hq.gemm(hq.FORMAT_TERNARY2, to_dev_u16(Xb, O.F16), Wp, S, N, group=256)
    torch.cuda.synchronize()
    ref = O.gemv_tq1_0(O.to_f32(Xb, O.F16), blocks, N)
    err = assert_parity(Y, ref, 1e-2, f"tq1_0 M={M} K={K} N={N}")
    assert err <= 2e-3, err  # fp16 output rounding bound
    assert np.all(np.isfinite(to_host_f32(Y)))  # non-finite d blocks are dropped, not propagated
