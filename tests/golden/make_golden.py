"""Writes tests/golden/qgemm_small.npz: small qGEMM cases with float64 expected outputs.

Inputs come from numpy's generator and numpy/torch rounding, and the expected Y is a
float64 numpy matmul of an independent numpy dequantisation ((q - 8) * s for int4,
t * s for ternary). Nothing here calls the oracle or the HIP library, so the file
pins both. Run from the repository root: python tests/golden/make_golden.py
"""
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "qgemm_small.npz"


def bf16_bits(x: np.ndarray) -> np.ndarray:
    import torch

    return torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def bf16_value(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def case(rng, fmt, xdtype, M, K, N, g):
    x = rng.standard_normal((M, K))
    if xdtype == 1:
        X = x.astype(np.float16).view(np.uint16)
        xv = X.view(np.float16).astype(np.float64)
    else:
        X = bf16_bits(x)
        xv = bf16_value(X).astype(np.float64)
    s = np.abs(rng.standard_normal((K // g, N)) * 0.02).astype(np.float16)
    sv = np.repeat(s.astype(np.float64), g, axis=0)
    if fmt == 1:
        q = rng.integers(0, 16, size=(K, N), dtype=np.uint32)
        W = np.bitwise_or.reduce(q.reshape(K // 8, 8, N) << (4 * np.arange(8, dtype=np.uint32))[None, :, None],
                                 axis=1).astype(np.uint32)
        wv = (q.astype(np.float64) - 8.0) * sv
    else:
        c = rng.choice(np.array([0, 1, 2], dtype=np.uint32), size=(K, N), p=[0.25, 0.5, 0.25])
        W = np.bitwise_or.reduce(c.reshape(K // 16, 16, N) << (2 * np.arange(16, dtype=np.uint32))[None, :, None],
                                 axis=1).astype(np.uint32)
        wv = (c.astype(np.float64) - 1.0) * sv
    return {"fmt": fmt, "xdtype": xdtype, "group": g, "N": N, "X": X, "W": W.ravel(),
            "scales": s.view(np.uint16), "Y64": xv @ wv}


def main():
    rng = np.random.default_rng(20260101)
    cases = {
        "int4_f16": case(rng, 1, 1, 4, 256, 32, 128),
        "int4_bf16": case(rng, 1, 2, 3, 384, 40, 128),
        "tern_bf16": case(rng, 2, 2, 5, 256, 48, 128),
        "tern_f16": case(rng, 2, 1, 2, 512, 24, 256),
        "int4_f16_m16_n20": case(rng, 1, 1, 16, 512, 20, 128),
    }
    flat = {f"{name}/{k}": np.asarray(v) for name, d in cases.items() for k, v in d.items()}
    np.savez_compressed(OUT, **flat)
    print(OUT, sum(v.nbytes for v in flat.values()), "bytes")


if __name__ == "__main__":
    main()
