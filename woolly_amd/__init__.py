"""woolly_amd -- MI355X (gfx950) backend for woolly's quantized matmul hot path.

The product is libwoolly_hip.so (hand-written HIP kernels behind the C ABI in
include/woolly_hip.h).  This package builds it (build.py), binds it with
ctypes (_lib.py), and mirrors the reference's Rust API on top of it
(quantization.py, gguf.py) plus device-level entry points (ops.py, device.py)
and the seeded synthetic-input generator of the benchmark (synth.py).
"""
from . import _lib
from ._lib import WoollyHipError

__all__ = ["WoollyHipError", "load_library"]


def load_library():
    """Loads libwoolly_hip.so; raises if it was not built (no CPU fallback)."""
    return _lib.load()
