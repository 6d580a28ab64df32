"""Split-fuse row assembly of nebula_amd.decoder (CPU: pure host logic on CPU tensors).

The order follows the reference batcher (hydrogen/src/batcher/split_fuse.cpp:110-159):
decode chunks (one token each) first, then the prefill chunk."""
import pytest
import torch

from nebula_amd.decoder import Chunk, StepRows, SHAPES, FUSED_GROUPS


def test_step_rows_order_and_split():
    chunks = [Chunk(7, 40, 64, True), Chunk(3, 12, 1, False), Chunk(5, 99, 1, False)]
    rows = StepRows(chunks)
    assert [c.request_id for c in rows.chunks] == [3, 5, 7]
    assert rows.offsets == [0, 1, 2] and rows.M == 66
    src = {3: torch.full((1, 4), 3.0), 5: torch.full((1, 4), 5.0), 7: torch.arange(64.0).repeat(4, 1).T.contiguous()}
    X = rows.gather(src)
    assert X.shape == (66, 4)
    assert torch.equal(X[0], src[3][0]) and torch.equal(X[1], src[5][0]) and torch.equal(X[2:], src[7])
    back = rows.split(X * 2)
    assert torch.equal(back[7], src[7] * 2) and torch.equal(back[3], src[3] * 2)


def test_step_rows_rejects_bad_chunks():
    with pytest.raises(ValueError):
        StepRows([Chunk(1, 0, 2, False)])  # a decode chunk holds one token
    rows = StepRows([Chunk(1, 0, 3, True)])
    with pytest.raises(ValueError):
        rows.gather({1: torch.zeros(2, 4)})


def test_projection_table_matches_reference_launches():
    # native_decoder.cu:1113-1115, 1141, 1149-1150, 1162, 1178-1179, 1183 with the 27B dimensions.
    assert SHAPES["attn_q"] == (5120, 12288) and SHAPES["attn_k"] == SHAPES["attn_v"] == (5120, 1024)
    assert SHAPES["attn_output"] == SHAPES["ssm_out"] == (6144, 5120)
    assert SHAPES["ssm_gate"] == (5120, 6144) and SHAPES["ssm_qkv"] == (5120, 10240)
    assert SHAPES["ffn_gate"] == SHAPES["ffn_up"] == (5120, 17408) and SHAPES["ffn_down"] == (17408, 5120)
    for kind, (fused, single) in FUSED_GROUPS.items():
        assert len({SHAPES[n][0] for n in fused}) == 1, kind  # a fused group shares its input
        assert all(SHAPES[n][0] % 256 == 0 for n in fused + single)
