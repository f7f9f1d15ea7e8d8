"""Seeded synthetic inputs: N(0, sigma) f32 tensors and their GGUF quantization.

Thin ctypes layer over libyule_synth.so (yule_amd/csrc/synth.c).  Same seed
-> same bytes on every host of this image; the quantizers are deterministic
but not parity-critical (GPU and CPU consume the same bytes).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

from .formats import DType, matrix_bytes

LIB_PATH = Path(__file__).resolve().parent / "libyule_synth.so"
_lib = None


def _load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(f"{LIB_PATH} is not built: run `python -m yule_amd.build`")
        lib = C.CDLL(str(LIB_PATH))
        lib.ys_gauss.argtypes = [C.c_uint64, C.c_float, C.c_size_t, C.c_size_t, C.c_void_p]
        lib.ys_gauss.restype = None
        lib.ys_uniform_u32.argtypes = [C.c_uint64, C.c_uint32, C.c_size_t, C.c_void_p]
        lib.ys_uniform_u32.restype = None
        lib.ys_f32_to_f16.argtypes = [C.c_float]
        lib.ys_f32_to_f16.restype = C.c_uint16
        lib.ys_quantize.argtypes = [C.c_int, C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p]
        lib.ys_quantize.restype = C.c_int
        lib.ys_gen_quant.argtypes = [C.c_int, C.c_uint64, C.c_float, C.c_size_t, C.c_size_t, C.c_void_p]
        lib.ys_gen_quant.restype = C.c_int
        _lib = lib
    return _lib


def gauss(seed: int, shape, sigma: float = 1.0) -> np.ndarray:
    """f32 array of `shape` ~ N(0, sigma^2); row r (last axis) uses stream r."""
    shape = (shape,) if isinstance(shape, int) else tuple(shape)
    n_cols = shape[-1] if shape else 1
    n_rows = int(np.prod(shape[:-1])) if len(shape) > 1 else 1
    out = np.empty(shape, dtype=np.float32)
    _load().ys_gauss(seed, sigma, n_rows, n_cols, out.ctypes.data)
    return out


def uniform_tokens(seed: int, n: int, vocab: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    _load().ys_uniform_u32(seed, vocab, n, out.ctypes.data)
    return out


def f32_to_f16_bits(v: float) -> int:
    return int(_load().ys_f32_to_f16(v))


def quantize(dtype: DType, x: np.ndarray) -> np.ndarray:
    """Quantize a 2-D f32 matrix into raw GGUF block bytes (u8, row-major)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        x = x[None, :]
    n_rows, n_cols = x.shape
    out = np.empty(matrix_bytes(dtype, n_rows, n_cols), dtype=np.uint8)
    if _load().ys_quantize(int(dtype), x.ctypes.data, n_rows, n_cols, out.ctypes.data):
        raise ValueError("quantize failed")
    return out


def gen_quant(dtype: DType, seed: int, n_rows: int, n_cols: int, sigma: float = 0.02) -> np.ndarray:
    """gauss(seed, (n_rows, n_cols), sigma) quantized, without the f32 copy."""
    out = np.empty(matrix_bytes(dtype, n_rows, n_cols), dtype=np.uint8)
    if _load().ys_gen_quant(int(dtype), seed, sigma, n_rows, n_cols, out.ctypes.data):
        raise ValueError("gen_quant failed")
    return out
