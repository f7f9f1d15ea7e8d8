"""Pins of the CPU oracle (oracle/*.c) — run on CPU, no GPU needed.

Each oracle function is checked against something other than its own
formula: the reference's known-answer tests (tests/golden/reference_kats.json),
the reference's own hand-written Q4_K AVX2 assembly (built from the
reference sources into oracle/_ref/; its outputs on the reference's xorshift
blocks are also committed as tests/golden/q4k_asm_vectors.npz), exhaustive
bit-pattern sweeps, packers written from the block layouts (round trips),
closed-form special cases, and brute-force f64 dots.
"""
import math

import numpy as np
import pytest

import oracle
from refgen import (GOLDEN, kats, pack_q4k, pack_q4k_scales, pack_q6k, q6k_sub_of, tolerance_bar, xorshift_blocks)
from yule_amd import DType, synth

K = kats()
RNG = np.random.default_rng(1234)


def hexb(s: str) -> np.ndarray:
    return np.frombuffer(bytes.fromhex(s), dtype=np.uint8).copy()


# ------------------------------------------------------------------ f16
def test_f16_kats():
    for bits, want in K["f16_to_f32"]["cases"]:
        assert oracle.f16_to_f32(bits) == want


def test_f16_exhaustive_vs_ieee():
    """All 65536 patterns against numpy's IEEE half -> single conversion."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(want) | np.isinf(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    nan = np.isnan(want)
    assert np.isnan(got[nan]).all()
    # dequant.rs:41-43 keeps the NaN payload bits (mant << 13), sign included
    exp = ((bits[nan].astype(np.uint32) & 0x8000) << 16) | 0x7F800000 | ((bits[nan].astype(np.uint32) & 0x3FF) << 13)
    # (the value crosses ctypes as a C float -> Python float conversion, which
    # sets the quiet bit; every other payload bit must survive)
    q = np.uint32(0x00400000)
    assert np.array_equal(got[nan].view(np.uint32) | q, exp | q)


# ------------------------------------------------------------------ Q4_0 / Q8_0
def test_q4_0_kats():
    z = K["q4_0_zero_block"]
    assert np.all(np.abs(oracle.dequant(oracle.Q4_0, hexb(z["block_hex"]))) < z["tol"])
    it = K["q4_0_interleave"]
    out = oracle.dequant(oracle.Q4_0, hexb(it["block_hex"]))
    assert out[0] == it["expect_first"][0] and out[1] == it["expect_first"][1]
    vd = K["q4_0_vec_dot_ones"]
    assert abs(oracle.vec_dot(oracle.Q4_0, hexb(vd["block_hex"]), np.ones(32, np.float32)) - vd["expect"]) < vd["tol"]


def test_q8_0_kats():
    e = K["q8_0_extremes"]
    out = oracle.dequant(oracle.Q8_0, hexb(e["block_hex"]))
    assert list(out[:2]) == e["expect_first"]
    d = K["q8_0_dispatch"]
    assert oracle.dequant(oracle.Q8_0, hexb(d["block_hex"]))[0] == d["expect_first"][0]


@pytest.mark.parametrize("d_bits", [0x3C00, 0x3800, 0x2E66, 0xB400, 0x0001, 0x7BFF])
def test_q4_0_q8_0_bruteforce(d_bits):
    """Every byte value at every position, against (nib-8)*d / (i8)q*d in f32."""
    d = np.float32(np.uint16(d_bits).view(np.float16))
    for v in range(256):
        b4 = np.zeros(18, np.uint8); b4[0:2] = np.frombuffer(np.uint16(d_bits).tobytes(), np.uint8); b4[2:] = v
        out = oracle.dequant(oracle.Q4_0, b4)
        lo, hi = np.float32((v & 15) - 8) * d, np.float32((v >> 4) - 8) * d
        assert np.array_equal(out, np.tile(np.array([lo, hi], np.float32), 16))
        b8 = np.zeros(34, np.uint8); b8[0:2] = b4[0:2]; b8[2:] = v
        assert np.array_equal(oracle.dequant(oracle.Q8_0, b8), np.full(32, np.float32(np.int8(np.uint8(v))) * d))


# ------------------------------------------------------------------ Q4_K
def test_q4k_scale_extraction_roundtrip():
    """extract(pack(sc, mn)) == (sc, mn) for random and boundary 6-bit values."""
    cases = [np.zeros(8, np.uint8), np.full(8, 63, np.uint8), np.arange(8, dtype=np.uint8) * 9]
    cases += [RNG.integers(0, 64, 8).astype(np.uint8) for _ in range(2000)]
    for sc in cases:
        mn = RNG.integers(0, 64, 8).astype(np.uint8)
        gsc, gmn = oracle.extract_q4k_scales_mins(pack_q4k_scales(sc, mn))
        assert np.array_equal(gsc, sc) and np.array_equal(gmn, mn)


def test_q4k_scale_extraction_bit_probe():
    """Each of the 96 scale bits moves exactly one (scale|min, bit) output."""
    seen = set()
    for byte in range(12):
        for bit in range(8):
            q = np.zeros(12, np.uint8)
            q[byte] = 1 << bit
            sc, mn = oracle.extract_q4k_scales_mins(q)
            nz = [("sc", i, int(v)) for i, v in enumerate(sc) if v] + [("mn", i, int(v)) for i, v in enumerate(mn) if v]
            assert len(nz) == 1 and bin(nz[0][2]).count("1") == 1
            seen.add((nz[0][0], nz[0][1], nz[0][2]))
    assert len(seen) == 96


def test_q4k_special_cases():
    q = RNG.integers(0, 16, 256)
    ones = np.ones(8, np.uint8)
    # d=1, sc=1, dmin=0 -> raw nibble levels
    out = oracle.dequant(oracle.Q4_K, pack_q4k(0x3C00, 0, ones, np.zeros(8, np.uint8), q))
    assert np.array_equal(out, q.astype(np.float32))
    # scale 0, mins only -> constant -dmin*mn per sub-block
    mn = np.arange(1, 9, dtype=np.uint8)
    out = oracle.dequant(oracle.Q4_K, pack_q4k(0x3C00, 0x3800, np.zeros(8, np.uint8), mn, q))
    assert np.array_equal(out, np.repeat(-0.5 * mn.astype(np.float32), 32))
    # distinct scales: weight i uses sub-block i // 32
    sc = np.arange(1, 9, dtype=np.uint8)
    out = oracle.dequant(oracle.Q4_K, pack_q4k(0x3C00, 0, sc, np.zeros(8, np.uint8), q))
    assert np.array_equal(out, q * np.repeat(sc, 32).astype(np.float32))


def test_q4k_dequant_vs_reference_asm_one_hot():
    """The reference's own assembly kernel (q4k_gemv_avx2.S) dotted with one-hot
    activations returns each dequantized weight: (d*sc)*q - (dmin*mn)."""
    asm = oracle.q4k_asm()
    if asm is None:
        pytest.skip("oracle/_ref not built (reference tree absent); vectors pinned by the .npz test")
    for blk, _ in xorshift_blocks("q4_k", 8):
        deq = oracle.dequant(oracle.Q4_K, blk)
        for i in range(256):
            e = np.zeros(256, np.float32); e[i] = 1.0
            got = asm(blk.ctypes.data, e.ctypes.data)
            assert math.isclose(got, deq[i], rel_tol=2e-7, abs_tol=1e-6), (i, got, deq[i])


def test_q4k_vec_dot_vs_reference_asm():
    """vec_dot_q4_k (scalar and AVX2 restatements) vs the reference assembly on
    the reference's xorshift blocks; asm outputs committed as golden vectors."""
    data = np.load(GOLDEN / "q4k_asm_vectors.npz")
    blocks, acts, want = data["blocks"], data["acts"], data["asm_dot"]
    asm = oracle.q4k_asm()
    for i in range(len(blocks)):
        if asm is not None:
            assert asm(blocks[i].ctypes.data, acts[i].ctypes.data) == want[i]
        s = oracle.vec_dot(oracle.Q4_K, blocks[i], acts[i], scalar=True)
        v = oracle.vec_dot(oracle.Q4_K, blocks[i], acts[i], scalar=False)
        f64 = float(np.dot(oracle.dequant(oracle.Q4_K, blocks[i]).astype(np.float64), acts[i].astype(np.float64)))
        tol = 1e-4 * max(1.0, abs(f64))
        assert abs(s - want[i]) < tol and abs(v - want[i]) < tol and abs(s - f64) < tol


# ------------------------------------------------------------------ Q6_K
def test_q6k_special_cases():
    q = RNG.integers(0, 64, 256)
    # d=1, all scales 1 -> q - 32
    out = oracle.dequant(oracle.Q6_K, pack_q6k(0x3C00, np.ones(16, np.int8), q))
    assert np.array_equal(out, (q - 32).astype(np.float32))
    # distinct (signed) scales identify the sub-block each weight uses
    sc = np.array([1, -2, 3, -4, 5, -6, 7, -8, 9, -10, 11, -12, 13, -14, 15, -16], np.int8)
    out = oracle.dequant(oracle.Q6_K, pack_q6k(0x3800, sc, q))
    want = np.array([0.5 * sc[q6k_sub_of(i)] * (q[i] - 32) for i in range(256)], np.float32)
    assert np.array_equal(out, want)


def test_q6k_bit_probe():
    """Flipping one quant bit in ql/qh moves exactly one output weight."""
    base = pack_q6k(0x3C00, np.ones(16, np.int8), np.full(256, 32))
    ref = oracle.dequant(oracle.Q6_K, base)
    hit = set()
    for byte in range(192):
        for bit in range(8):
            b = base.copy(); b[byte] ^= 1 << bit
            diff = np.nonzero(oracle.dequant(oracle.Q6_K, b) != ref)[0]
            assert len(diff) == 1
            hit.add(int(diff[0]))
    assert hit == set(range(256))


def test_q6k_vec_dot_vs_f64():
    for blk, act in xorshift_blocks("q6_k", 200):
        f64 = float(np.dot(oracle.dequant(oracle.Q6_K, blk).astype(np.float64), act.astype(np.float64)))
        for scalar in (True, False):
            assert abs(oracle.vec_dot(oracle.Q6_K, blk, act, scalar) - f64) < 1e-3 * max(1.0, abs(f64))


# ------------------------------------------------------------------ Q5_K
def q5k_from_q4k(q4: np.ndarray, qh: np.ndarray) -> np.ndarray:
    """Q5_K block with a Q4_K block's header and quants plus 32 qh bytes
    (layouts: dequant.rs:255-290 vs :292-338)."""
    b = np.zeros(176, np.uint8)
    b[0:16] = q4[0:16]
    b[16:48] = qh
    b[48:176] = q4[16:144]
    return b


def test_q5k_reference_kat():
    k = K["q5_k_dequant"]
    b = np.zeros(176, np.uint8)
    b[0:2] = hexb(k["d_hex"])
    b[2:4] = hexb(k["dmin_hex"])
    b[4] = k["scale0_byte"]
    b[48] = k["qs48"]
    assert oracle.dequant(oracle.Q5_K, b)[0] == k["expect_w0"]
    b[16] = 1
    assert oracle.dequant(oracle.Q5_K, b)[0] == k["qh16_bit0_expect_w0"]


def test_q5k_without_high_bits_is_q4k():
    """With qh = 0 a Q5_K block is exactly the Q4_K block of the same header
    and quants (both dequant and vec_dot); the 5th bits then add exactly
    16 * d * sc to one weight each: bit b of qh[l] moves only weight
    64*(b//2) + 32*(b%2) + l."""
    for blk4, act in xorshift_blocks("q4_k", 40):
        b5 = q5k_from_q4k(blk4, np.zeros(32, np.uint8))
        ref = oracle.dequant(oracle.Q4_K, blk4)
        assert np.array_equal(oracle.dequant(oracle.Q5_K, b5).view(np.uint32), ref.view(np.uint32))
        assert oracle.vec_dot(oracle.Q5_K, b5, act, True) == oracle.vec_dot(oracle.Q4_K, blk4, act, True)
    blk4 = next(xorshift_blocks("q4_k", 1))[0]
    d = oracle.f16_to_f32(int(blk4[0]) | (int(blk4[1]) << 8))
    sc, _ = oracle.extract_q4k_scales_mins(blk4[4:16])
    base = q5k_from_q4k(blk4, np.zeros(32, np.uint8))
    ref = oracle.dequant(oracle.Q5_K, base).astype(np.float64)
    for l in (0, 7, 31):
        for bit in range(8):
            b = base.copy()
            b[16 + l] |= 1 << bit
            diff = oracle.dequant(oracle.Q5_K, b).astype(np.float64) - ref
            idx = np.nonzero(diff)[0]
            w = 64 * (bit // 2) + 32 * (bit % 2) + l
            assert list(idx) == [w], (l, bit, idx)
            assert abs(diff[w] - 16.0 * d * float(sc[bit])) <= 1e-6 * max(1.0, abs(ref[w]) + 16 * d * sc[bit])


def test_q5k_vec_dot_vs_f64():
    for blk, act in xorshift_blocks("q5_k", 200):
        f64 = float(np.dot(oracle.dequant(oracle.Q5_K, blk).astype(np.float64), act.astype(np.float64)))
        for scalar in (True, False):
            assert abs(oracle.vec_dot(oracle.Q5_K, blk, act, scalar) - f64) < 1e-3 * max(1.0, abs(f64))


# ------------------------------------------------------------------ Q8_K
@pytest.mark.parametrize("d", [1.0, 0.5, -0.03125, 3.0e-8, 1.0e30, 2.0 ** -149])
def test_q8k_closed_form(d):
    """Every int8 value at several f32 scales: w = (i8)q * d (dequant.rs:376-384);
    the bsums tail is not read; there is no Q8_K vec_dot (simd/scalar.rs:4-22)."""
    b = np.zeros(292, np.uint8)
    b[0:4] = np.frombuffer(np.float32(d).tobytes(), np.uint8)
    b[4:260] = np.arange(256, dtype=np.uint8)
    want = (np.arange(256, dtype=np.uint8).view(np.int8).astype(np.float32) * np.float32(d)).astype(np.float32)
    got = oracle.dequant(oracle.Q8_K, b)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    b[260:292] = 0xAB
    assert np.array_equal(oracle.dequant(oracle.Q8_K, b).view(np.uint32), want.view(np.uint32))
    with pytest.raises(ValueError):
        oracle.vec_dot(oracle.Q8_K, b, np.ones(256, np.float32))


@pytest.mark.parametrize("fmt,dt", [("q8_0", oracle.Q8_0), ("q4_0", oracle.Q4_0), ("q4_k", oracle.Q4_K),
                                    ("q5_k", oracle.Q5_K), ("q6_k", oracle.Q6_K)])
def test_avx2_vs_scalar_reference_generators(fmt, dt):
    """The reference's differential tests (avx2.rs:346-573), same seeds and tolerances."""
    g = K["xorshift_generators"][fmt]
    n = min(g["iters"], 2000)
    for blk, act in xorshift_blocks(fmt, n):
        s = oracle.vec_dot(dt, blk, act, scalar=True)
        v = oracle.vec_dot(dt, blk, act, scalar=False)
        assert abs(s - v) < g["tol"]


# ------------------------------------------------------------------ qmv / argmax / rope
def test_qmv_two_row_kat():
    k = K["q4_0_qmm_two_rows"]
    w = np.concatenate([hexb(k["weights_hex"]), hexb(k["weights_hex_row1"])])
    x = np.full(32, k["input"], np.float32)
    for y in (oracle.qmv_scalar(oracle.Q4_0, w, x, 2, 32), oracle.qmv(oracle.Q4_0, w, x, 2, 32)):
        assert np.all(np.abs(y - np.array(k["expect"])) < k["tol"])


@pytest.mark.parametrize("dt", [oracle.Q4_0, oracle.Q8_0, oracle.Q4_K, oracle.Q5_K, oracle.Q6_K])
def test_qmv_threaded_matches_f64(dt):
    """Threaded AVX2 qmv and the single-thread scalar qmv vs f64 dots (300 rows,
    so the >=128-row thread split is exercised)."""
    from yule_amd import synth
    bs, bb = oracle.GEOM[dt]
    n_rows, n_cols = 300, 4 * 256
    w = synth.gen_quant(dt, 7, n_rows, n_cols)
    x = synth.gauss(8, n_cols)
    ref = oracle.qmv_f64(dt, w, x, n_rows, n_cols)
    bar = 1e-3 * np.linalg.norm(ref) / np.sqrt(n_rows)
    assert np.max(np.abs(oracle.qmv(dt, w, x, n_rows, n_cols, 4) - ref)) < bar
    assert np.max(np.abs(oracle.qmv_scalar(dt, w, x, n_rows, n_cols) - ref)) < bar


def test_argmax_kats():
    a = K["argmax"]
    assert oracle.argmax(np.array(a["values"], np.float32)) == a["expect"]
    # ties: the last maximal index wins (ct_gte keeps v >= best)
    assert oracle.argmax(np.array([1.0, 3.0, 3.0, 2.0], np.float32)) == 2
    assert oracle.argmax(np.array([5.0, 5.0, 5.0], np.float32)) == 2
    assert oracle.argmax(np.array([-np.inf, -1.0], np.float32)) == 1
    v = RNG.standard_normal(32000).astype(np.float32)
    assert oracle.argmax(v) == int(np.argmax(v))


def test_argmax_infinite_ties():
    """argmax_ct's test is the sign bit of (v - best) (sampler.rs:142-148).
    inf - inf is the IEEE default NaN, which x86 produces with the sign bit
    set, so an equal infinity never replaces the best: the first of several
    +inf wins, and an all -inf input stays at index 0."""
    inf = np.inf
    nan = np.float32(inf) - np.float32(inf)
    assert np.signbit(nan)          # the x86 default NaN this rule rests on
    for vals, want in (([inf, 1.0, inf], 0), ([-inf] * 5, 0), ([1.0, inf, 2.0, inf], 1),
                       ([-inf, 3.0, 3.0], 2), ([2.0, -inf], 0), ([-inf, -inf, 0.5, -inf], 2)):
        assert oracle.argmax(np.array(vals, np.float32)) == want, vals


def test_rope_table_kats():
    c, s = oracle.rope_table(8, 4, 10000.0)
    assert np.all(c[:2] == 1.0) and np.all(s[:2] == 0.0)
    # pos 5, pair 0: freq 1 -> theta 5 (cpu.rs:771-790)
    assert abs(c[5 * 2] - math.cos(5.0)) < 1e-6 and abs(s[5 * 2] - math.sin(5.0)) < 1e-6
    # pair 1: freq = 1/10000^(2/4) = 0.01
    assert abs(c[5 * 2 + 1] - math.cos(0.05)) < 1e-6


def test_qmv_through_reference_asm_matches_restatement():
    """oracle.set_q4k_dot(q4k_asm()): the AVX2 qmv with the reference's own
    assembly block dot (the reference's AVX2 build) agrees with the
    Rust-fallback restatement and with the f64 dot, threaded and not."""
    asm = oracle.q4k_asm()
    if asm is None:
        pytest.skip("oracle/_ref not built (needs the reference tree)")
    w = synth.gen_quant(DType.Q4_K, 61, 300, 4096)
    x = synth.gauss(62, 4096)
    ref = oracle.qmv_f64(int(DType.Q4_K), w, x, 300, 4096)
    port = oracle.qmv(int(DType.Q4_K), w, x, 300, 4096, 4)
    oracle.set_q4k_dot(asm)
    try:
        a1 = oracle.qmv(int(DType.Q4_K), w, x, 300, 4096, 1)
        a4 = oracle.qmv(int(DType.Q4_K), w, x, 300, 4096, 4)
    finally:
        oracle.set_q4k_dot(None)
    assert np.array_equal(a1, a4)
    assert np.max(np.abs(a1 - ref)) <= tolerance_bar(ref)
    assert np.max(np.abs(a1 - port)) <= tolerance_bar(ref)
    assert np.array_equal(oracle.qmv(int(DType.Q4_K), w, x, 300, 4096, 4), port)   # restored
