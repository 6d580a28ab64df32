"""The reference decoder's projections as fused qGEMM calls, for any number of rows.

hydrogen's native decoder (hydrogen/src/model/native_decoder.cu:1097-1198) runs every
projection of a layer as its own `kernel_gemv_tq1_0` launch over one token's fp32 activation
(M = 1; prompt tokens go through one at a time, :1297), re-reading the shared input once per
projection. Here a layer's TQ1_0 weights are imported once (hq_repack_tq1_0_device) and the
projections that share an input run as one fused call over all rows of a step:

    attention layer  q | k | v  (5120 -> 12288 | 1024 | 1024)   :1113-1115  one fused call
                     attn_output (6144 -> 5120)                  :1141
    SSM layer        gate | qkv (5120 -> 6144 | 10240)           :1149-1150  one fused call
                     ssm_out (6144 -> 5120)                      :1162
    FFN              gate | up  (5120 -> 17408 | 17408)          :1178-1179  one fused call
                     down (17408 -> 5120)                        :1183

Rows are independent, so a step's rows may be any mix of decode tokens and prefill tokens
(the split-fuse batch of hydrogen/src/batcher/split_fuse.cpp:110-159: the decode streams'
tokens first, then one prefill chunk); the library picks its streaming (decode) kernels for
up to 80 rows and its prefill kernels above. `StepRows` builds such a batch's activation
matrix and splits the outputs back per chunk. Normalisation, attention, the SSM step and SwiGLU stay with the
caller: they are not projections.

Activations are fp16 or bf16 (the reference's are fp32); the ternary weights and their
per-block scales are kept exactly (group = 256, one scale per TQ1_0 block).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

from . import hq

# Dimensions of the reference's 27B model (hydrogen/include/native_decoder.hpp:180-188).
EMBEDDING = 5120
FFN = 17408
Q_OUT = 12288
KV_OUT = 1024
MIXER_IN = 6144      # attn_output / ssm_out input width
SSM_GATE = 6144
SSM_QKV = 10240
TQ1_GROUP = 256

# Projection name -> (K, N), as the reference launches them.
SHAPES: Dict[str, Tuple[int, int]] = {
    "attn_q": (EMBEDDING, Q_OUT), "attn_k": (EMBEDDING, KV_OUT), "attn_v": (EMBEDDING, KV_OUT),
    "attn_output": (MIXER_IN, EMBEDDING),
    "ssm_gate": (EMBEDDING, SSM_GATE), "ssm_qkv": (EMBEDDING, SSM_QKV), "ssm_out": (MIXER_IN, EMBEDDING),
    "ffn_gate": (EMBEDDING, FFN), "ffn_up": (EMBEDDING, FFN), "ffn_down": (FFN, EMBEDDING),
}
# Projections that read the same input and run as one call.
FUSED_GROUPS = {
    "attention": (("attn_q", "attn_k", "attn_v"), ("attn_output",)),
    "ssm": (("ssm_gate", "ssm_qkv"), ("ssm_out",)),
    "ffn": (("ffn_gate", "ffn_up"), ("ffn_down",)),
}


@dataclass
class TernaryProjection:
    """One imported TQ1_0 projection: packed ternary tiles and fp16 scales [K/256, N]."""
    K: int
    N: int
    Wp: object
    S: object

    @classmethod
    def from_tq1_0(cls, blocks, K: int, N: int, stream=None) -> "TernaryProjection":
        """blocks: the GGUF tensor's bytes on the device (N rows of K/256 56-byte blocks)."""
        Wp, S = hq.repack_tq1_0_device(blocks, K, N, stream=stream)
        return cls(K, N, Wp, S)


class LayerProjections:
    """The projections of one decoder layer (attention or SSM mixer, plus the FFN)."""

    def __init__(self, kind: str, weights: Dict[str, TernaryProjection]):
        if kind not in ("attention", "ssm"):
            raise ValueError(f"layer kind must be 'attention' or 'ssm', got {kind!r}")
        self.kind = kind
        need = [n for grp in FUSED_GROUPS[kind] + FUSED_GROUPS["ffn"] for n in grp]
        for name in need:
            if name not in weights:
                raise KeyError(f"{kind} layer needs weight {name!r}")
            if (weights[name].K, weights[name].N) != SHAPES[name]:
                raise ValueError(f"{name}: shape {(weights[name].K, weights[name].N)}, expected {SHAPES[name]}")
        self.w = weights

    def _fused(self, names: Sequence[str], X, outs=None, stream=None):
        segs = [(self.w[n].Wp, self.w[n].S, self.w[n].N) for n in names]
        return hq.gemm_fused(hq.FORMAT_TERNARY2, X, segs, TQ1_GROUP, outs=outs, stream=stream)

    def mixer_in(self, x_norm, outs=None, stream=None) -> List:
        """Attention: [q, k, v]; SSM: [gate, qkv] — one fused call over all rows."""
        return self._fused(FUSED_GROUPS[self.kind][0], x_norm, outs, stream)

    def mixer_out(self, y, out=None, stream=None):
        """attn_output or ssm_out (6144 -> 5120)."""
        return self._fused(FUSED_GROUPS[self.kind][1], y, None if out is None else [out], stream)[0]

    def ffn_in(self, x_norm, outs=None, stream=None) -> List:
        """[gate, up] — one fused call."""
        return self._fused(FUSED_GROUPS["ffn"][0], x_norm, outs, stream)

    def ffn_out(self, act, out=None, stream=None):
        """down (17408 -> 5120)."""
        return self._fused(FUSED_GROUPS["ffn"][1], act, None if out is None else [out], stream)[0]


@dataclass
class Chunk:
    """A slice of one request's tokens in a step (hydrogen/include/batcher.hpp:47-52)."""
    request_id: int
    start_token: int
    num_tokens: int
    is_prefill: bool


class StepRows:
    """The activation rows of one split-fuse step, in the batcher's order (decode chunks, then
    the prefill chunk), and the way back from output rows to chunks."""

    def __init__(self, chunks: Sequence[Chunk]):
        ordered = [c for c in chunks if not c.is_prefill] + [c for c in chunks if c.is_prefill]
        self.chunks = ordered
        self.offsets = []
        m = 0
        for c in ordered:
            if c.num_tokens < 1 or (not c.is_prefill and c.num_tokens != 1):
                raise ValueError(f"bad chunk {c}: decode chunks hold one token, prefill chunks at least one")
            self.offsets.append(m)
            m += c.num_tokens
        self.M = m

    def gather(self, rows_of: Dict[int, object], out=None):
        """rows_of[request_id]: that request's activations for this step's tokens
        ([num_tokens, K] device tensor). Returns X [M, K]."""
        import torch

        parts = [rows_of[c.request_id] for c in self.chunks]
        for c, p in zip(self.chunks, parts):
            if p.shape[0] != c.num_tokens:
                raise ValueError(f"request {c.request_id}: {p.shape[0]} rows, chunk has {c.num_tokens}")
        if out is None:
            return torch.cat(parts, dim=0)
        torch.cat(parts, dim=0, out=out)
        return out

    def split(self, Y) -> Dict[int, object]:
        """Output rows back per request (views into Y)."""
        return {c.request_id: Y[o:o + c.num_tokens] for c, o in zip(self.chunks, self.offsets)}


def random_tq1_0(K: int, N: int, generator=None, device="cuda"):
    """Synthetic TQ1_0 bytes of an N x K projection: uniform trit bytes, d = |N(0, 0.02)| fp16."""
    import torch

    nb = K // 256
    raw = torch.randint(0, 256, (N * nb, 56), dtype=torch.uint8, device=device, generator=generator)
    d = (torch.randn(N * nb, device=device, generator=generator).abs() * 0.02).to(torch.float16)
    raw[:, 0:2] = d.view(torch.uint8).view(N * nb, 2)
    raw[:, 54:56] = 0
    return raw.reshape(-1)


def random_layer(kind: str, generator=None, device="cuda") -> LayerProjections:
    names = [n for grp in FUSED_GROUPS[kind] + FUSED_GROUPS["ffn"] for n in grp]
    w = {}
    for n in names:
        K, N = SHAPES[n]
        w[n] = TernaryProjection.from_tq1_0(random_tq1_0(K, N, generator, device), K, N)
    return LayerProjections(kind, w)
