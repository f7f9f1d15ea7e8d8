"""Input generators of the reference's own differential tests, and
independent helpers the oracle tests use.

`xorshift_blocks` reproduces the block/activation streams of
yule-core/src/simd/avx2.rs:346-573 (Q5_K: :510-540) (xorshift64 <<13 >>7 <<17, fixed headers,
activations (r % 1000)/500 - 1) so parity runs on the same inputs the
reference's AVX2-vs-scalar tests use.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"
M64 = (1 << 64) - 1


def kats() -> dict:
    return json.loads((GOLDEN / "reference_kats.json").read_text())


class XorShift:
    def __init__(self, seed: int):
        self.s = seed & M64

    def next(self) -> int:
        s = self.s
        s ^= (s << 13) & M64
        s ^= s >> 7
        s ^= (s << 17) & M64
        self.s = s
        return s

    def act(self, n: int) -> np.ndarray:
        return np.array([(self.next() % 1000) / 500.0 - 1.0 for _ in range(n)], dtype=np.float32)


def xorshift_blocks(fmt: str, count: int):
    """Yield (block u8[], act f32[]) exactly as avx2.rs's tests build them."""
    if fmt == "q8_0":
        g = XorShift(42)
        for _ in range(count):
            b = np.zeros(34, np.uint8)
            b[0], b[1] = 0x00, 0x38
            for i in range(32):
                b[2 + i] = g.next() & 0xFF
            yield b, g.act(32)
    elif fmt == "q4_0":
        g = XorShift(123)
        for _ in range(count):
            b = np.zeros(18, np.uint8)
            b[0], b[1] = 0x00, 0x38
            for i in range(16):
                b[2 + i] = g.next() & 0xFF
            yield b, g.act(32)
    elif fmt == "q4_k":
        g = XorShift(777)
        for _ in range(count):
            b = np.zeros(144, np.uint8)
            b[0], b[1], b[2], b[3] = 0x00, 0x38, 0x66, 0x2E
            for i in range(4, 144):
                b[i] = g.next() & 0xFF
            for i in range(4, 16):
                b[i] = g.next() % 64
            yield b, g.act(256)
    elif fmt == "q5_k":
        g = XorShift(888)
        for _ in range(count):
            b = np.zeros(176, np.uint8)
            b[0], b[1], b[2], b[3] = 0x00, 0x38, 0x66, 0x2E
            for i in range(4, 176):
                b[i] = g.next() & 0xFF
            for i in range(4, 16):
                b[i] = g.next() % 64
            yield b, g.act(256)
    elif fmt == "q6_k":
        g = XorShift(999)
        for _ in range(count):
            b = np.zeros(210, np.uint8)
            for i in range(210):
                b[i] = g.next() & 0xFF
            b[208], b[209] = 0x00, 0x38
            for i in range(192, 208):
                b[i] = g.next() % 20
            yield b, g.act(256)
    else:
        raise ValueError(fmt)


# ---- independent packers, written from the GGUF/ggml block layouts ----------
# (the inverse direction of the dequantizers, so a wrong index in either
# side breaks the round trip)

def pack_q4k_scales(sc, mn) -> np.ndarray:
    """ggml Q4_K 12-byte scale packing: scales/mins 0-3 in the low 6 bits of
    bytes 0-3 / 4-7; for 4-7 the low 4 bits go to the low/high nibble of
    bytes 8-11 and the top 2 bits to bits 6-7 of bytes 0-3 / 4-7."""
    q = np.zeros(12, np.uint8)
    for j in range(4):
        q[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        q[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        q[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return q


def pack_q4k(d_bits: int, dmin_bits: int, sc, mn, q256) -> np.ndarray:
    """Q4_K block from 8 scales, 8 mins and 256 4-bit levels (weight order)."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(d_bits).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.uint16(dmin_bits).tobytes(), np.uint8)
    b[4:16] = pack_q4k_scales(sc, mn)
    q = np.asarray(q256, np.uint8)
    for j in range(4):
        b[16 + 32 * j:48 + 32 * j] = q[64 * j:64 * j + 32] | (q[64 * j + 32:64 * j + 64] << 4)
    return b


def pack_q6k(d_bits: int, scales16, q256) -> np.ndarray:
    """Q6_K block from 16 int8 scales and 256 unsigned 6-bit levels: per half
    of 128, ql[l] = q[l] | q[l+64]<<4, ql[l+32] = q[l+32] | q[l+96]<<4,
    qh[l] = hi2(q[l]) | hi2(q[l+32])<<2 | hi2(q[l+64])<<4 | hi2(q[l+96])<<6."""
    b = np.zeros(210, np.uint8)
    q = np.asarray(q256, np.int64)
    for h in range(2):
        qq = q[128 * h:128 * h + 128]
        for l in range(32):
            q1, q2, q3, q4 = qq[l], qq[l + 32], qq[l + 64], qq[l + 96]
            b[64 * h + l] = (q1 & 15) | ((q3 & 15) << 4)
            b[64 * h + 32 + l] = (q2 & 15) | ((q4 & 15) << 4)
            b[128 + 32 * h + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    b[192:208] = np.asarray(scales16, np.int8).view(np.uint8)
    b[208:210] = np.frombuffer(np.uint16(d_bits).tobytes(), np.uint8)
    return b


def q6k_sub_of(i: int) -> int:
    """Index of the int8 scale that weight i of a Q6_K block uses."""
    h, r = divmod(i, 128)
    g, l = divmod(r, 32)
    return 8 * h + l // 16 + 2 * g


def tolerance_bar(y_ref: np.ndarray) -> float:
    """The matvec parity bar: max|y - y_ref| <= 1e-3 * ||y_ref||_2 / sqrt(N)."""
    y = np.asarray(y_ref, np.float64)
    return 1e-3 * float(np.linalg.norm(y)) / np.sqrt(max(1, y.size))
