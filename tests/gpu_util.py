"""Helpers for GPU parity tests: move oracle-generated host arrays to the device and back."""
from __future__ import annotations

import numpy as np

import oracle as O
from nebula_amd import hq


def to_dev_u16(a: np.ndarray, dtype: int | None = None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()
    if dtype == O.F16:
        return t.view(torch.float16)
    if dtype == O.BF16:
        return t.view(torch.bfloat16)
    return t


def to_dev_u32(a: np.ndarray):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).cuda()


def to_host_f32(y) -> np.ndarray:
    import torch

    return y.float().cpu().numpy() if y.dtype != torch.float32 else y.cpu().numpy()


class DeviceProblem:
    """An oracle Problem with its packed weight, scales and activations resident on the GPU."""

    def __init__(self, P: O.Problem):
        self.P = P
        self.X = to_dev_u16(P.X, P.xdtype)
        self.S = to_dev_u16(P.scales)
        self.packed_host = hq.repack(P.fmt, P.W, P.K, P.N)
        self.Wp = to_dev_u32(self.packed_host)

    def run(self, out=None, X=None):
        return hq.gemm(self.P.fmt, self.X if X is None else X, self.Wp, self.S, self.P.N, self.P.group, out=out)


def assert_parity(y_dev, ref: np.ndarray, tol: float = 1e-2, label: str = "") -> float:
    """normwise max relative error <= 1e-2 (fp32 accumulation on both sides)."""
    y = to_host_f32(y_dev)
    assert y.shape == ref.shape, (y.shape, ref.shape)
    assert np.all(np.isfinite(y)), f"{label}: non-finite outputs"
    err = O.normwise_error(y, ref)
    assert err <= tol, f"{label}: normwise error {err:.3e} > {tol}"
    return err
