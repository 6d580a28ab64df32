"""GPU parity over seeded random shapes, each planned by the library's default planner.

The parametrised tests elsewhere pin each kernel and tiling on chosen shapes; these cases draw
(format, activation dtype, M, K, N, group, bias) at random from a fixed seed so that the
planner's choices are exercised on shapes nobody picked: M over the three bands (1-16: the
X-resident / per-wavefront kernels, 17-80: the lockstep kernel's row tiles, 81-300: the prefill
tiles, whole and stream-K), ragged N (1..3000), K up to 6144 in multiples of 128 and of the
group, groups 32 / 64 (general kernels) and 128 / 256, and the int4 caller bias. Each case is
checked against the oracle with the bars of the general-kernel tests: normwise error within the
output rounding (2e-3 fp16, 8e-3 bf16) and, per element, |y - r| <= rel * |X| (|W| + |E|) +
ulp(r) (rel = 2^-10 fp16, 2^-7 bf16; E the weight of code 8 of each int4 group). A second set
draws wide decode calls (M 1-16, N 24576-32768) that the planner streams in slab pairs, a third
long-K decode calls (K 8192-32768) that it cuts into K pieces, a fourth prefill calls of
301-2048 rows.
"""
import numpy as np
import pytest

import oracle as O
from test_gpu_general import Dev, check

pytestmark = pytest.mark.gpu

MAX_MACS = 1.2e9  # keeps the oracle and the float64 bound check to about a second a case


def _cases(n: int = 96, seed: int = 20261202):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        fmt = (O.INT4, O.TERNARY2)[i % 2]
        xdt = (O.F16, O.BF16)[(i // 2) % 2]
        band = (i // 4) % 3
        lo, hi = ((1, 16), (17, 80), (81, 300))[band]
        M = int(rng.integers(lo, hi + 1))
        group = int(rng.choice([32, 64, 128, 256]))
        step = 256 if group == 256 else 128  # K: a multiple of 128 and of the group
        K = step * int(rng.integers(1, 6144 // step + 1))
        N = int(rng.integers(1, 3001))
        N = max(1, min(N, int(MAX_MACS // (M * K))))
        bias = "random" if fmt == O.INT4 and rng.random() < 0.5 else None
        cases.append((fmt, xdt, M, K, N, group, bias, 9000 + i))
    return cases


CASES = _cases()


@pytest.mark.parametrize("fmt,xdt,M,K,N,group,bias,seed", CASES,
                         ids=[f"f{c[0]}-d{c[1]}-M{c[2]}-K{c[3]}-N{c[4]}-g{c[5]}-{c[6] or 'nobias'}" for c in CASES])
def test_random_shape(cuda, fmt, xdt, M, K, N, group, bias, seed):
    P = O.Problem(fmt, M, K, N, group, xdt, seed=seed, bias=bias)
    label = f"fmt={fmt} dt={xdt} M={M} K={K} N={N} g={group} bias={bias} seed={seed}"
    print(label, flush=True)
    check(Dev(P).run(), P, label)


def _wide_cases(n: int = 16, seed: int = 20261203):
    # Wide decode calls whose 4-tile slabs number 1.5 to 2 times the CUs (N = 24576..32768 on
    # 256 CUs): the default planner streams them in slab pairs (int4 at any M, ternary above
    # eight rows), with an odd slab count leaving the last workgroup one slab.
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        fmt = (O.INT4, O.TERNARY2)[i % 2]
        xdt = (O.F16, O.BF16)[(i // 2) % 2]
        M = int(rng.integers(1, 17))
        group = int(rng.choice([128, 256]))
        K = 256 * int(rng.integers(1, 9))
        N = int(rng.integers(24576, 32769))
        cases.append((fmt, xdt, M, K, N, group, 9500 + i))
    return cases


WIDE = _wide_cases()


@pytest.mark.parametrize("fmt,xdt,M,K,N,group,seed", WIDE,
                         ids=[f"f{c[0]}-d{c[1]}-M{c[2]}-K{c[3]}-N{c[4]}-g{c[5]}" for c in WIDE])
def test_random_wide_decode(cuda, fmt, xdt, M, K, N, group, seed):
    import torch

    from nebula_amd import hq

    P = O.Problem(fmt, M, K, N, group, xdt, seed=seed)
    desc = hq.describe(fmt, xdt, M, K, N, group=group)
    label = f"fmt={fmt} dt={xdt} M={M} K={K} N={N} g={group} seed={seed}: {desc}"
    print(label, flush=True)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert (",SG=2>" in desc) == (fmt == O.INT4 or M > 8), label
    check(Dev(P).run(), P, label)


def _long_k_cases(n: int = 16, seed: int = 20261204):
    # Long K at decode row counts: rows of all of K that do not fit in LDS at several rows, so
    # the planner cuts K into pieces (X-resident, even and uneven, up to eight rows; lockstep
    # above, with four k-groups where each gets eight or more steps), N ragged.
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        fmt = (O.INT4, O.TERNARY2)[i % 2]
        xdt = (O.F16, O.BF16)[(i // 2) % 2]
        M = int(rng.integers(1, 17))
        group = int(rng.choice([128, 256]))
        K = 256 * int(rng.integers(32, 129))
        N = int(rng.integers(64, 6001))
        N = max(64, min(N, int(MAX_MACS // (M * K))))
        cases.append((fmt, xdt, M, K, N, group, 9700 + i))
    return cases


LONG_K = _long_k_cases()


@pytest.mark.parametrize("fmt,xdt,M,K,N,group,seed", LONG_K,
                         ids=[f"f{c[0]}-d{c[1]}-M{c[2]}-K{c[3]}-N{c[4]}-g{c[5]}" for c in LONG_K])
def test_random_long_k_decode(cuda, fmt, xdt, M, K, N, group, seed):
    from nebula_amd import hq

    P = O.Problem(fmt, M, K, N, group, xdt, seed=seed)
    label = f"fmt={fmt} dt={xdt} M={M} K={K} N={N} g={group} seed={seed}: {hq.describe(fmt, xdt, M, K, N, group=group)}"
    print(label, flush=True)
    check(Dev(P).run(), P, label)


def _prefill_cases(n: int = 8, seed: int = 20261205):
    # Prefill row counts past the random band above (301-2048 rows): 64-, 128- and 256-row tiles,
    # the half-height tail launch and stream-K as the planner picks them, ragged N.
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        fmt = (O.INT4, O.TERNARY2)[i % 2]
        xdt = (O.F16, O.BF16)[(i // 2) % 2]
        M = int(rng.integers(301, 2049))
        group = int(rng.choice([64, 128, 256])) if fmt == O.INT4 else int(rng.choice([128, 256]))
        K = 256 * int(rng.integers(4, 7))
        N = int(rng.integers(2048, 8193)) if i % 3 else int(rng.integers(256, 2049))
        N = max(256, min(N, int(1e10 // (M * K))))
        bias = "random" if fmt == O.INT4 and i % 4 == 0 else None
        cases.append((fmt, xdt, M, K, N, group, bias, 9800 + i))
    return cases


PREFILL = _prefill_cases()


@pytest.mark.parametrize("fmt,xdt,M,K,N,group,bias,seed", PREFILL,
                         ids=[f"f{c[0]}-d{c[1]}-M{c[2]}-K{c[3]}-N{c[4]}-g{c[5]}-{c[6] or 'nobias'}" for c in PREFILL])
def test_random_prefill(cuda, fmt, xdt, M, K, N, group, bias, seed):
    from nebula_amd import hq

    P = O.Problem(fmt, M, K, N, group, xdt, seed=seed, bias=bias)
    desc = hq.describe(fmt, xdt, M, K, N, group=group, with_bias=bias is not None)
    label = f"fmt={fmt} dt={xdt} M={M} K={K} N={N} g={group} bias={bias} seed={seed}: {desc}"
    print(label, flush=True)
    check(Dev(P).run(), P, label)
