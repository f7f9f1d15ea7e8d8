"""yule_amd — MI355X (gfx950) HIP backend for Yule's quantized matmul path.

The product is libyule_hip.so (C ABI in include/yule_hip.h); `HipBackend`
mirrors Yule's ComputeBackend trait over it.  No CPU fallback exists: without
the built library or a gfx950 device every entry point raises.
"""
from .formats import DType, GEOMETRY, block_bytes, block_size, matrix_bytes, row_bytes  # noqa: F401

__all__ = ["DType", "GEOMETRY", "block_bytes", "block_size", "matrix_bytes", "row_bytes", "HipBackend",
           "YuleGpuError", "BufferHandle", "load_library"]


def __getattr__(name):
    if name in ("HipBackend", "YuleGpuError", "BufferHandle", "load_library", "is_available"):
        from . import backend
        return getattr(backend, name)
    raise AttributeError(name)
