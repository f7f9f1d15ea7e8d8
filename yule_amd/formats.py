"""GGUF block formats on the hot path (yule-core/src/dtype.rs:13-118)."""
from __future__ import annotations

from enum import IntEnum


class DType(IntEnum):
    """GGUF type ids, dtype.rs:21-35 (the values cross the C ABI)."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q8_0 = 8
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15


# (weights per block, bytes per block): dtype.rs:62-118
GEOMETRY = {
    DType.Q4_0: (32, 18),
    DType.Q8_0: (32, 34),
    DType.Q4_K: (256, 144),
    DType.Q5_K: (256, 176),
    DType.Q6_K: (256, 210),
    DType.Q8_K: (256, 292),
}
QUANTIZED = tuple(GEOMETRY)


def block_size(dt: DType) -> int:
    return GEOMETRY[DType(dt)][0]


def block_bytes(dt: DType) -> int:
    return GEOMETRY[DType(dt)][1]


def row_bytes(dt: DType, n_cols: int) -> int:
    bs, bb = GEOMETRY[DType(dt)]
    if n_cols % bs:
        raise ValueError(f"n_cols {n_cols} is not a multiple of {bs} for {DType(dt).name}")
    return n_cols // bs * bb


def matrix_bytes(dt: DType, n_rows: int, n_cols: int) -> int:
    return n_rows * row_bytes(dt, n_cols)
