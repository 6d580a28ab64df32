"""CPU check of the decode work decomposition (stream-K ranges, pieces, fix-up slots).

tests/plan_check.cpp includes the same header the kernel uses (nebula_amd/csrc/hq_plan.hpp)
and walks every workgroup and wavefront of many (slabs, k-blocks, workgroups, wavefronts)
combinations; it is compiled here with g++ and run as a subprocess.
"""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_decode_plan_covers_every_unit_once(tmp_path):
    exe = tmp_path / "plan_check"
    subprocess.run(
        ["g++", "-O2", "-std=c++17", f"-I{ROOT / 'nebula_amd' / 'csrc'}", str(ROOT / "tests" / "plan_check.cpp"),
         "-o", str(exe)],
        check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.startswith("ok"), out.stdout
