"""diagpu_amd -- MI355X (gfx950) diagonal-format sparse kernels.

The product is libdiagpu.so (HIP kernels behind the C ABI of
include/diagpu.h).  This package locates it and gives Python callers
(tests, bench.py) a thin ctypes view over torch device tensors.
"""
from ._lib import DiagpuError, load  # noqa: F401

__all__ = ["DiagpuError", "load"]
