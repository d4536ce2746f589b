"""sfnx_amd: the quantized mixture-of-experts hot path of sFNX, MI355X-native (gfx950 HIP kernels behind a C ABI).

The compute lives in libsfnx_moe.so (include/sfnx_moe.h); this package binds it.  Importing the package does not load
the library; the first call does, and raises if it is not built.
"""
from ._abi import LIB_PATH, Q4_K, Q8_0, lib  # noqa: F401

__all__ = ["LIB_PATH", "Q4_K", "Q8_0", "lib"]
