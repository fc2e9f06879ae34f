"""e4b -- Python host for libe4b.so, the MI355X (gfx950) batch-1 decode library.

Mirrors the reference engine's host surface (src/engine-a4b.js, src/gguf.js)
over the C ABI in include/e4b.h.  Importing this package loads the HIP
library; there is no CPU fallback.
"""
from ._lib import LIB_PATH, E4BError, check, last_error, lib  # noqa: F401
from . import device, formats, kernels  # noqa: F401

__all__ = ["LIB_PATH", "E4BError", "check", "last_error", "lib", "device", "formats", "kernels"]
