"""ffai_amd — MI355X (gfx950) mixture-of-experts layer for FFAI.

The product is libmoehip.so (C ABI in include/moe_hip.h, HIP kernels in
ffai_amd/csrc). This package holds its build step and the ctypes view of the
ABI used by tests and bench.py; ffai_amd.layer wraps a layer around PyTorch
device buffers.
"""
from ._lib import load, check, last_error, MoeError, LIB_PATH  # noqa: F401

__all__ = ["load", "check", "last_error", "MoeError", "LIB_PATH"]
