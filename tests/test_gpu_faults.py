"""Failure reporting of kernels that give up a bounded wait, forced from the host.

The lockstep decode kernel's k-group barrier and the barrier of the two K halves of a prefill
tile (KS = 2) poll an LDS arrival count a bounded number of times. HQ_DECODE_LS_SPIN=0 makes
every wait give up at once: the wavefronts carry on (so the kernel exits normally, with wrong
outputs) and set the host-visible fault word, which the next hq_device_status() (or the next
GEMM call) reports as HQ_ERR_DEVICE and clears.
"""
import os

import pytest

import oracle as O
from gpu_util import DeviceProblem
from nebula_amd import hq

pytestmark = pytest.mark.gpu


def test_kgroup_barrier_timeout_is_reported(cuda):
    # 20 rows: only the lockstep kernel takes them, with two k-groups (the barrier is used).
    P = O.Problem(O.INT4, 20, 2048, 1024, 128, O.F16, seed=9100)
    D = DeviceProblem(P)
    assert "KG=2" in hq.describe(O.INT4, O.F16, 20, 2048, 1024)
    D.run()
    hq.device_status()  # no fault so far
    os.environ["HQ_DECODE_LS_SPIN"] = "0"
    try:
        D.run()
    finally:
        del os.environ["HQ_DECODE_LS_SPIN"]
    with pytest.raises(hq.HQError) as ei:
        hq.device_status()
    assert ei.value.status == hq.HQ_ERR_DEVICE and "k-group barrier" in ei.value.message
    hq.device_status()  # the word was cleared
    # A GEMM call also reports a pending fault before launching anything.
    os.environ["HQ_DECODE_LS_SPIN"] = "0"
    try:
        D.run()
    finally:
        del os.environ["HQ_DECODE_LS_SPIN"]
    import torch

    torch.cuda.synchronize()
    with pytest.raises(hq.HQError) as ei:
        D.run()
    assert ei.value.status == hq.HQ_ERR_DEVICE
    # Afterwards calls run and are right again.
    y = D.run()
    hq.device_status()
    from test_gpu_parity import check

    check(y, P.reference(), O.F16, "after a reported fault", P)


def test_prefill_k_halves_barrier_timeout_is_reported(cuda):
    # A prefill tile split in two K halves of one workgroup meets per k-block at an LDS
    # arrival count; giving up is reported like the decode k-group barrier.
    from test_gpu_parity import check, prefill_env

    P = O.Problem(O.INT4, 300, 2048, 1000, 128, O.F16, seed=9110)
    D = DeviceProblem(P)
    with prefill_env(KS=2, WM=1, SK=0, TAIL=0):
        assert "k-split in workgroup" in hq.describe(O.INT4, O.F16, 300, 2048, 1000)
        D.run()
        hq.device_status()  # no fault so far
        os.environ["HQ_DECODE_LS_SPIN"] = "0"
        try:
            D.run()
        finally:
            del os.environ["HQ_DECODE_LS_SPIN"]
        with pytest.raises(hq.HQError) as ei:
            hq.device_status()
        assert ei.value.status == hq.HQ_ERR_DEVICE and "K halves" in ei.value.message
        hq.device_status()  # the word was cleared
        y = D.run()
        hq.device_status()
    check(y, P.reference(), O.F16, "prefill after a reported fault", P)
