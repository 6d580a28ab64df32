"""nebula_amd — MI355X (gfx950) weight-only quantized GEMM for hydrogen's qGEMM path.

The compute lives in libnebula_hq.so (HIP, built by nebula_amd.build); this package
holds its ctypes binding (nebula_amd.hq) and the build recipe.
"""
from . import hq  # noqa: F401

__all__ = ["hq"]
