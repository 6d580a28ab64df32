"""CPU-only build of the host code under AddressSanitizer + UndefinedBehaviorSanitizer.

The kernels are built as usual (nebula_amd/build.py); the sources with host logic (argument
validation, host repacks, TQ1_0 and Q4_K conversion, the GGUF parser) are compiled again with
the sanitizers on their host pass only and linked with the regular kernel objects into
nebula_amd/lib/libnebula_hq_san.so; the oracle gets a sanitized twin (oracle/Makefile.san)
built with the same clang runtime, so both share one runtime in a process.
tests/test_sanitizers.py runs the CPU test suites against both with that runtime preloaded.
Nothing here runs on a GPU.
"""
from __future__ import annotations

import os
from pathlib import Path

from .build import ARCH, BUILD, COMMON_FLAGS, CSRC, HIPCC, LIBDIR, ORACLE_DIR, SOURCES, _run

SAN_LIB = LIBDIR / "libnebula_hq_san.so"
SAN_HOST = ["-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=undefined",
            "-fno-omit-frame-pointer", "-shared-libsan", "-g"]
SAN_SOURCES = ["hq_api.cpp", "hq_gguf.cpp"]
LLVM = Path(os.environ.get("HQ_LLVM", "/opt/rocm/llvm"))


def asan_runtime() -> Path:
    """clang's shared ASan runtime (to preload into an uninstrumented python)."""
    hits = sorted(LLVM.glob("lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not hits:
        raise RuntimeError(f"no libclang_rt.asan-x86_64.so under {LLVM}")
    return hits[-1]


def build_sanitized() -> tuple[Path, Path]:
    BUILD.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    host = [f for flag in SAN_HOST for f in ("-Xarch_host", flag)]
    objs = []
    for src in SOURCES:
        if src in SAN_SOURCES:
            obj = BUILD / (src + ".san.o")
            _run([HIPCC, "-x", "hip", *COMMON_FLAGS, *host, "-c", str(CSRC / src), "-o", str(obj)])
        else:
            obj = BUILD / (src + ".o")
            if not obj.exists():
                _run([HIPCC, "-x", "hip", *COMMON_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(obj)
    tmp = SAN_LIB.with_suffix(".so.tmp")
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *host, *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, SAN_LIB)
    _run(["make", "-C", str(ORACLE_DIR), "-s", "-f", "Makefile.san", f"LLVM={LLVM}"])
    return SAN_LIB, ORACLE_DIR / "liboracle_hq_san.so"




if __name__ == "__main__":
    print(*build_sanitized())
