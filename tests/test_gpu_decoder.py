"""GPU tests of nebula_amd.decoder: a layer's projections (the reference decoder's
kernel_gemv_tq1_0 launches, hydrogen/src/model/native_decoder.cu:1113-1183) imported from
TQ1_0 and run as fused calls over M rows match the oracle's restatement of kernel_gemv_tq1_0
on the same blocks (normwise 1e-2 bar, fp16 output bound 2e-3), on a spot check of rows at
the 27B shapes; a split-fuse step (decode tokens + a prefill chunk in one call) equals running
each request on its own."""
import numpy as np
import pytest

import oracle as O
from gpu_util import to_host_f32
from nebula_amd import decoder as D
from nebula_amd import hq

pytestmark = pytest.mark.gpu


def host_layer(kind, seed):
    import torch

    blocks, w = {}, {}
    names = [n for grp in D.FUSED_GROUPS[kind] + D.FUSED_GROUPS["ffn"] for n in grp]
    for i, n in enumerate(names):
        K, N = D.SHAPES[n]
        blocks[n] = O.gen_tq1_0(seed + i, N, K, nonfinite_every=97)
        w[n] = D.TernaryProjection.from_tq1_0(torch.from_numpy(blocks[n].reshape(-1)).cuda(), K, N)
    return D.LayerProjections(kind, w), blocks


def check_rows(Y, Xb, blocks, N, rows, label):
    ref = O.gemv_tq1_0(O.to_f32(Xb[rows], O.F16), blocks, N, threads=16)
    err = O.normwise_error(to_host_f32(Y)[rows], ref)
    assert err <= 2e-3, f"{label}: normwise {err:.3e}"


@pytest.mark.parametrize("kind", ["attention", "ssm"])
@pytest.mark.parametrize("M", [1, 16, 80, 300])
def test_layer_projections_match_gemv(cuda, kind, M):
    import torch

    L, blocks = host_layer(kind, 4000 + M)
    rng = np.random.default_rng(M)
    rows = np.sort(rng.choice(M, size=min(M, 2), replace=False))
    fused_in, (single,) = D.FUSED_GROUPS[kind]
    X = O.gen_normal(M, 1, M * D.EMBEDDING, 1.0, False, O.F16).reshape(M, D.EMBEDDING)
    outs = L.mixer_in(torch.from_numpy(X.view(np.int16)).cuda().view(torch.float16))
    for n, Y in zip(fused_in, outs):
        check_rows(Y, X, blocks[n], D.SHAPES[n][1], rows, f"{kind} {n} M={M}")
    Xo = O.gen_normal(M, 2, M * D.MIXER_IN, 1.0, False, O.F16).reshape(M, D.MIXER_IN)
    Y = L.mixer_out(torch.from_numpy(Xo.view(np.int16)).cuda().view(torch.float16))
    check_rows(Y, Xo, blocks[single], D.EMBEDDING, rows, f"{kind} {single} M={M}")
    if kind == "attention":  # the FFN is the same for both layer kinds
        gate, up = L.ffn_in(torch.from_numpy(X.view(np.int16)).cuda().view(torch.float16))
        check_rows(gate, X, blocks["ffn_gate"], D.FFN, rows, f"ffn_gate M={M}")
        check_rows(up, X, blocks["ffn_up"], D.FFN, rows, f"ffn_up M={M}")
        Xa = O.gen_normal(M, 3, M * D.FFN, 1.0, False, O.F16).reshape(M, D.FFN)
        Y = L.ffn_out(torch.from_numpy(Xa.view(np.int16)).cuda().view(torch.float16))
        check_rows(Y, Xa, blocks["ffn_down"], D.EMBEDDING, rows, f"ffn_down M={M}")


def test_split_fuse_step_equals_separate_requests(cuda):
    import torch

    g = torch.Generator(device="cuda").manual_seed(5)
    L = D.random_layer("attention", generator=g)
    chunks = [D.Chunk(i + 1, 100 + i, 1, False) for i in range(16)] + [D.Chunk(99, 0, 64, True)]
    rows = D.StepRows(chunks)
    src = {c.request_id: torch.randn((c.num_tokens, D.EMBEDDING), device="cuda", generator=g).half()
           for c in chunks}
    X = rows.gather(src)
    assert rows.M == 80
    fused = [rows.split(y) for y in L.mixer_in(X)]  # one call: 80 rows, prefill kernels
    for c in chunks:
        alone = L.mixer_in(src[c.request_id])  # 1 row (decode kernels) or 64 rows
        for i, y in enumerate(alone):
            err = O.normwise_error(to_host_f32(fused[i][c.request_id]), to_host_f32(y))
            assert err <= 2e-3, (c, i, err)
