"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

nebula_amd/build_sanitize.py builds libnebula_hq_san.so (argument validation, host repacks,
TQ1_0 and Q4_K conversion and the GGUF parser instrumented; the kernels as usual) and the
oracle's sanitized twin with one clang runtime; this test runs the CPU suites against both in
a child process with that runtime preloaded, failing on the first report (halt_on_error). The
GGUF tests parse every prefix of a file and malformed headers, the ABI tests pass invalid
enums, null pointers and bad shapes, so the parsers and validators see hostile input here.
"""
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
SUITES = ["tests/test_abi.py", "tests/test_gguf.py", "tests/test_oracle.py", "tests/test_rust_binding.py"]


def test_cpu_suites_under_asan_and_ubsan():
    sys.path.insert(0, str(ROOT))
    from nebula_amd import build_sanitize as BS

    lib, olib = BS.build_sanitized()
    env = dict(os.environ, HQ_LIB=str(lib), HQO_LIB=str(olib), LD_PRELOAD=str(BS.asan_runtime()),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1", UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    proc = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", *SUITES,
                           "-m", "not gpu"], cwd=str(ROOT), env=env, capture_output=True, text=True, timeout=900)
    out = proc.stdout + proc.stderr
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert proc.returncode == 0, out[-4000:]
    assert " passed" in proc.stdout
