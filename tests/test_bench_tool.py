"""The BENCH-compatible executable (nebula_amd/bin/hq_bench_qgemm), driven like the reference's
hydrogen/tests/test_h08_marlin_gemm.py drives hydrogen_bench_marlin_gemm: same options, same
JSON keys, same sweep and invariants. The reference's >= 80% bus-utilisation gate is
reported, not asserted: the tool measures with weights rotated past the Infinity Cache, and
the MI355X decode target is tracked by bench.py.
"""
import json
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
EXE = ROOT / "nebula_amd" / "bin" / "hq_bench_qgemm"


def run_tool(args, timeout=120):
    return subprocess.run([str(EXE)] + args, capture_output=True, text=True, cwd=str(ROOT), timeout=timeout)


def test_bench_tool_binary_exists():
    assert EXE.exists(), f"not built: {EXE} (run nebula_amd/build.py)"


def test_bench_tool_help():
    proc = run_tool(["--help"])
    assert proc.returncode == 0
    for flag in ("Usage:", "--json", "--k", "--n", "--group", "--iters", "--warmups"):
        assert flag in proc.stdout


def check_status(data, proc):
    gates = [data["repack_under_1s"], data["numerical_match_passed"], data["latency_le_0_15ms_passed"],
             data["speedup_gt_1_8x_passed"]]
    if data["K"] >= 4096 and data["N"] >= 4096:
        gates.append(data["bandwidth_gt_80pct_passed"])
    assert data["status"] == ("PASS" if all(gates) else "FAIL")
    assert proc.returncode == (0 if data["status"] == "PASS" else 1)


@pytest.mark.gpu
def test_bench_tool_sweep_and_invariants(cuda):
    proc = run_tool(["--json"])
    assert proc.returncode in (0, 1), proc.stderr
    data = json.loads(proc.stdout)
    check_status(data, proc)
    assert (data["K"], data["N"], data["group_size"]) == (4096, 4096, 128)
    assert data["repack_under_1s"] is True and data["repack_time_ms"] < 1000.0
    assert data["numerical_match_passed"] is True
    assert data["latency_le_0_15ms_passed"] is True
    assert data["speedup_gt_1_8x_passed"] is True
    assert data["weight_copies"] > 1
    sweep = data["sweep"]
    assert [r["M"] for r in sweep] == [1, 2, 4, 8]
    for r in sweep:
        assert r["normwise_error"] <= 1e-2
        assert r["marlin_latency_ms"] <= 0.15
        assert r["speedup_ratio"] > 1.8
        assert 0 < r["bandwidth_util_pct"] == pytest.approx(100 * r["bandwidth_gbs"] / 8000.0, abs=0.11)
    assert data["peak_bandwidth_util_pct"] == pytest.approx(max(r["bandwidth_util_pct"] for r in sweep), abs=0.11)


@pytest.mark.gpu
def test_bench_tool_custom_dims(cuda):
    proc = run_tool(["--k", "2048", "--n", "2048", "--iters", "10", "--json"])
    data = json.loads(proc.stdout)
    assert (data["K"], data["N"]) == (2048, 2048)
    assert data["status"] == "PASS" and proc.returncode == 0, proc.stdout
    assert data["numerical_match_passed"] is True and data["latency_le_0_15ms_passed"] is True


@pytest.mark.gpu
def test_bench_tool_ternary_bf16_decode_shape(cuda):
    proc = run_tool(["--format", "ternary2", "--dtype", "bf16", "--k", "5120", "--n", "27648", "--m", "1,8",
                     "--iters", "5", "--warmups", "2", "--json"])
    data = json.loads(proc.stdout)
    check_status(data, proc)
    assert (data["format"], data["dtype"]) == ("ternary2", "bf16")
    assert [r["M"] for r in data["sweep"]] == [1, 8]
    assert data["numerical_match_passed"] is True


@pytest.mark.gpu
def test_bench_tool_formatted_output(cuda):
    proc = run_tool(["--m", "1,16", "--iters", "5"])
    assert proc.returncode in (0, 1), proc.stderr
    out = proc.stdout
    assert "Acceptance Criteria Verification:" in out
    assert "Weight Repacking (<1.0s):  PASS" in out
    assert "Numerical Accuracy (normwise <= 1e-2): PASS" in out
    assert "Overall Status:" in out
