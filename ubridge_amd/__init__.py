"""ubridge_amd -- MI355X (gfx950) drop-in for Ubridge's quantized-matmul path.

The compute lives in libubridge_hip.so (hand-written HIP kernels, C ABI in
include/ubridge_hip.h); this package is the host-side mirror of the
reference's operator interface.  Importing it loads the library and fails
loudly if it has not been built.
"""
from . import _lib  # noqa: F401  (raises ImportError when the .so is missing)
from .ops import *  # noqa: F401,F403
from .registry import get_function, has_function  # noqa: F401
from . import fp8, moe  # noqa: F401

__all__ = ["ops", "registry", "synth", "get_function", "has_function"]
