"""Build recipe for the gfx950 qGEMM library (libnebula_hq.so) and the CPU oracle.

The product library is compiled in-tree with hipcc for gfx950 only; objects go to
nebula_amd/_build/, the shared library to nebula_amd/lib/. Packed-fp32 VALU
instructions are disabled on purpose (-packed-fp32-ops): every kernel here is
written in scalar fp32 and packed fp16 arithmetic.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libnebula_hq.so"
BINDIR = PKG / "bin"
BENCH_TOOL = BINDIR / "hq_bench_qgemm"
STREAM_TOOL = BINDIR / "hq_stream_ceiling"
ORACLE_DIR = ROOT / "oracle"

SOURCES = ["hq_api.cpp", "hq_gguf.cpp", "hq_decode.hip", "hq_decode_ls.hip", "hq_prefill.hip", "hq_repack.hip", "hq_int8.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
    "-Wno-unknown-warning-option",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}")
    # hipcc's host pass does not know the packed-fp32 feature; that warning is expected.
    noise = ("packed-fp32-ops", "is not a recognized feature for this target")
    lines = [ln for ln in (proc.stdout + proc.stderr).splitlines() if not any(n in ln for n in noise)]
    if any(ln.strip() for ln in lines):
        sys.stderr.write("\n".join(lines) + "\n")


def build_library(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    procs = []
    objs = []
    for src in SOURCES:
        obj = BUILD / (src + ".o")
        lang = ["-x", "hip"]
        cmd = [HIPCC, *lang, *COMMON_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd))
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        objs.append(obj)
    failed = []
    for cmd, p in procs:
        out, _ = p.communicate()
        noise = ("packed-fp32-ops", "is not a recognized feature for this target")
        lines = [ln for ln in (out or "").splitlines() if not any(n in ln for n in noise)]
        if p.returncode != 0:
            failed.append((cmd, "\n".join(lines)))
        elif any(ln.strip() for ln in lines):
            sys.stderr.write("\n".join(lines) + "\n")
    if failed:
        for cmd, out in failed:
            sys.stderr.write(f"FAILED: {' '.join(cmd)}\n{out}\n")
        raise RuntimeError("HIP compilation failed")
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


def build_tools() -> Path:
    """The BENCH-compatible benchmark executable (links the library through its C ABI) and
    the stream-ceiling probe that bench.py runs beside the decode sweep."""
    BINDIR.mkdir(exist_ok=True)
    tmp = BENCH_TOOL.with_suffix(".tmp")
    _run([HIPCC, "-x", "hip", *COMMON_FLAGS, str(PKG / "tools" / "hq_bench_qgemm.cpp"), "-o", str(tmp),
          f"-L{LIBDIR}", "-lnebula_hq", "-Wl,-rpath,$ORIGIN/../lib"])
    os.replace(tmp, BENCH_TOOL)
    tmp = STREAM_TOOL.with_suffix(".tmp")
    _run([HIPCC, "-x", "hip", *COMMON_FLAGS, str(PKG / "tools" / "hq_stream_ceiling.hip"), "-o", str(tmp)])
    os.replace(tmp, STREAM_TOOL)
    return BENCH_TOOL


def build_oracle() -> Path:
    _run(["make", "-C", str(ORACLE_DIR), "-s"])
    return ORACLE_DIR / "liboracle_hq.so"


def build(verbose: bool = False) -> None:
    build_library(verbose)
    build_tools()
    build_oracle()


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(LIB)
