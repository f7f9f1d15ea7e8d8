"""GPU parity of the hot path through the C ABI: block dequant (bit-exact)
and quantized_matmul (max|y - y_ref| <= 1e-3 * ||y_ref||_2 / sqrt(N), y_ref
the f64-accumulated dot of the oracle's bit-exact dequantized weights; the
reference's own f32 CpuBackend result is checked against the same bar)."""
import sys

import numpy as np
import pytest

import oracle
from refgen import kats, tolerance_bar, xorshift_blocks
from yule_amd import DType, synth
from yule_amd.formats import block_size
from yule_amd.backend import YuleGpuError

pytestmark = pytest.mark.gpu

FMTS = [DType.Q4_0, DType.Q8_0, DType.Q4_K, DType.Q5_K, DType.Q6_K, DType.Q8_K]
# formats the reference's differential tests generate blocks for (avx2.rs:346-573)
XS_NAME = {DType.Q4_0: "q4_0", DType.Q8_0: "q8_0", DType.Q4_K: "q4_k", DType.Q5_K: "q5_k", DType.Q6_K: "q6_k"}
GEN_FMTS = list(XS_NAME)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.array_equal(a.view(np.uint32)[~nan], b.view(np.uint32)[~nan]) and
                np.array_equal(np.isnan(a), np.isnan(b)))


def gpu_dequant(hip, dt, data: np.ndarray, offset: int = 0) -> np.ndarray:
    bs, bb = oracle.GEOM[int(dt)]
    nb = (data.size - offset) // bb
    src = hip.upload(data)
    dst = hip.allocate(nb * bs * 4)
    hip.dequantize(src, offset, dst, nb, dt)
    out = hip.download(dst, nb * bs)
    hip.free(src); hip.free(dst)
    return out


def gpu_qmv(hip, dt, w, x, n_rows, n_cols) -> np.ndarray:
    hw, hx, hy = hip.upload(w), hip.upload(x), hip.allocate(n_rows * 4)
    hip.quantized_matmul(hw, hx, hy, n_rows, n_cols, dt)
    y = hip.download(hy, n_rows)
    for h in (hw, hx, hy):
        hip.free(h)
    return y


# ------------------------------------------------------------------ dequant
@pytest.mark.parametrize("dt", GEN_FMTS, ids=lambda d: d.name)
def test_dequant_bit_exact_reference_generators(hip, dt):
    say(f"[dequant] {dt.name} reference xorshift blocks")
    blocks = np.concatenate([b for b, _ in xorshift_blocks(XS_NAME[dt], 512)])
    assert same_bits(gpu_dequant(hip, dt, blocks), oracle.dequant(int(dt), blocks))


@pytest.mark.parametrize("dt", FMTS, ids=lambda d: d.name)
def test_dequant_bit_exact_random_bytes(hip, dt):
    """Uniformly random block bytes (every scale/min/quant pattern, any f16
    header incl. denormals, inf and NaN), at an odd block offset."""
    say(f"[dequant] {dt.name} random bytes")
    bs, bb = oracle.GEOM[int(dt)]
    rng = np.random.default_rng(int(dt))
    data = rng.integers(0, 256, bb * 4096 + bb, dtype=np.uint8)
    assert same_bits(gpu_dequant(hip, dt, data, offset=bb), oracle.dequant(int(dt), data[bb:]))


def test_dequant_reference_kats(hip):
    say("[dequant] reference KATs")
    k = kats()
    out = gpu_dequant(hip, DType.Q4_0, np.frombuffer(bytes.fromhex(k["q4_0_interleave"]["block_hex"]), np.uint8))
    assert out[0] == -8.0 and out[1] == 7.0
    out = gpu_dequant(hip, DType.Q8_0, np.frombuffer(bytes.fromhex(k["q8_0_extremes"]["block_hex"]), np.uint8))
    assert out[0] == 127.0 and out[1] == -128.0
    q5 = k["q5_k_dequant"]   # dequant.rs:1529-1563
    b = np.zeros(176, np.uint8)
    b[0:2] = np.frombuffer(bytes.fromhex(q5["d_hex"]), np.uint8)
    b[4], b[48] = q5["scale0_byte"], q5["qs48"]
    assert gpu_dequant(hip, DType.Q5_K, b)[0] == q5["expect_w0"]
    b[16] = 1
    assert gpu_dequant(hip, DType.Q5_K, b)[0] == q5["qh16_bit0_expect_w0"]


# ------------------------------------------------------------------ matvec
def test_qmv_reference_kat(hip):
    say("[qmv] cpu.rs 2-row Q4_0 KAT")
    k = kats()["q4_0_qmm_two_rows"]
    w = np.frombuffer(bytes.fromhex(k["weights_hex"] + k["weights_hex_row1"]), np.uint8)
    y = gpu_qmv(hip, DType.Q4_0, w, np.ones(32, np.float32), 2, 32)
    assert np.all(np.abs(y - 32.0) < k["tol"])


@pytest.mark.parametrize("dt", GEN_FMTS, ids=lambda d: d.name)
def test_qmv_reference_generator_rows(hip, dt):
    """Rows built from the reference's xorshift blocks and activations."""
    say(f"[qmv] {dt.name} xorshift rows")
    bs, bb = oracle.GEOM[int(dt)]
    pairs = list(xorshift_blocks(XS_NAME[dt], 256))
    per_row = 8
    n_rows = len(pairs) // per_row
    w = np.concatenate([b for b, _ in pairs])
    x = np.concatenate([a for _, a in pairs[:per_row]])
    n_cols = per_row * bs
    ref = oracle.qmv_f64(int(dt), w, x, n_rows, n_cols)
    y = gpu_qmv(hip, dt, w, x, n_rows, n_cols)
    assert np.max(np.abs(y - ref)) <= tolerance_bar(ref)


SHAPES = [(1, 256), (3, 512), (7, 1024), (33, 2048), (255, 2048), (257, 4096), (300, 5632), (64, 14336),
          (1000, 768), (4099, 256), (20, 20480), (9, 36864), (65, 11008)]


@pytest.mark.parametrize("dt", FMTS, ids=lambda d: d.name)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_qmv_shapes(hip, dt, shape):
    n_rows, n_cols = shape
    say(f"[qmv] {dt.name} {n_rows}x{n_cols}")
    w = synth.gen_quant(dt, 100 + n_rows, n_rows, n_cols)
    x = synth.gauss(200 + n_cols, n_cols)
    ref = oracle.qmv_f64(int(dt), w, x, n_rows, n_cols)
    y = gpu_qmv(hip, dt, w, x, n_rows, n_cols)
    bar = tolerance_bar(ref)
    assert np.max(np.abs(y - ref)) <= bar
    # the reference's own f32 path meets the same bar (sanity of the bar);
    # Q8_K has no vec_dot in the reference
    if dt != DType.Q8_K:
        assert np.max(np.abs(oracle.qmv_scalar(int(dt), w, x, n_rows, n_cols) - ref)) <= bar


def test_qmv_config0_full_size(hip):
    """Q4_0 5632x2048, W ~ N(0,0.02) seed 0, x ~ N(0,1)."""
    say("[qmv] config0 Q4_0 5632x2048")
    w = synth.gen_quant(DType.Q4_0, 0, 5632, 2048)
    x = synth.gauss(1, 2048)
    ref = oracle.qmv_f64(int(DType.Q4_0), w, x, 5632, 2048)
    y = gpu_qmv(hip, DType.Q4_0, w, x, 5632, 2048)
    assert np.max(np.abs(y - ref)) <= tolerance_bar(ref)


def test_qmv_rows_independent_and_linear(hip):
    """Size-independent properties at a large shape: y(a x1 + b x2) = a y(x1) + b y(x2)
    and each output row depends only on its own weight row."""
    say("[qmv] linearity Q4_K 14336x4096")
    dt, n_rows, n_cols = DType.Q4_K, 14336, 4096
    w = synth.gen_quant(dt, 5, n_rows, n_cols)
    x1, x2 = synth.gauss(6, n_cols), synth.gauss(7, n_cols)
    y1, y2 = gpu_qmv(hip, dt, w, x1, n_rows, n_cols), gpu_qmv(hip, dt, w, x2, n_rows, n_cols)
    y12 = gpu_qmv(hip, dt, w, (0.5 * x1 + 2.0 * x2).astype(np.float32), n_rows, n_cols)
    assert np.max(np.abs(y12 - (0.5 * y1 + 2.0 * y2))) <= 2 * tolerance_bar(y12)
    rows = [0, 1, 4095, 7777, 14335]
    sub = np.concatenate([w[r * 16 * 144:(r + 1) * 16 * 144] for r in rows])
    assert np.array_equal(gpu_qmv(hip, dt, sub, x1, len(rows), n_cols), y1[rows])


# BASELINE configs[2] (Llama-3-8B: FFN and the 128256-row lm_head, in each
# of the layer formats) and configs[1]'s Q6_K lm_head, at full size.
# configs[2]'s attention projections (Q/O 4096x4096, K/V 1024x4096) in each
# layer format, and configs[1]'s Q4_K TinyLlama projections as standalone
# matvecs.
FULL = [(dt, 14336, 4096) for dt in (DType.Q6_K, DType.Q8_0)] + \
       [(dt, 4096, 14336) for dt in (DType.Q4_K, DType.Q6_K, DType.Q8_0)] + \
       [(dt, 128256, 4096) for dt in (DType.Q4_K, DType.Q6_K, DType.Q8_0)] + [(DType.Q6_K, 32000, 2048)] + \
       [(dt, r, 4096) for dt in (DType.Q4_K, DType.Q6_K, DType.Q8_0) for r in (4096, 1024)] + \
       [(DType.Q4_K, r, c) for r, c in ((2048, 2048), (256, 2048), (5632, 2048), (2048, 5632))]


@pytest.mark.parametrize("dt,n_rows,n_cols", FULL, ids=lambda v: getattr(v, "name", str(v)))
def test_qmv_config_shapes_full_size(hip, dt, n_rows, n_cols):
    """The whole matrix on the GPU; every row up to 4096 rows, else 512
    seeded rows (first and last included), against the oracle's f64 dot of
    the same rows; and those rows run alone give bit-identical outputs (each
    row depends only on its own weights)."""
    say(f"[qmv] full size {dt.name} {n_rows}x{n_cols}")
    bs, bb = oracle.GEOM[int(dt)]
    row_bytes = n_cols // bs * bb
    w = synth.gen_quant(dt, 300 + int(dt), n_rows, n_cols)
    x = synth.gauss(301, n_cols)
    y = gpu_qmv(hip, dt, w, x, n_rows, n_cols)
    rows = np.arange(n_rows) if n_rows <= 4096 else np.unique(np.concatenate(
        [[0, n_rows - 1], np.random.default_rng(n_rows).integers(0, n_rows, 510)]))
    sub = np.concatenate([w[r * row_bytes:(r + 1) * row_bytes] for r in rows])
    ref = oracle.qmv_f64(int(dt), sub, x, len(rows), n_cols)
    assert np.max(np.abs(y[rows] - ref)) <= tolerance_bar(ref)
    assert np.array_equal(gpu_qmv(hip, dt, sub, x, len(rows), n_cols), y[rows])
    assert np.all(np.isfinite(y))


def test_qmv_edge_cases_and_errors(hip):
    say("[qmv] edge cases")
    dt = DType.Q4_K
    w = synth.gen_quant(dt, 9, 4, 256)
    x = synth.gauss(9, 256)
    hw, hx, hy = hip.upload(w), hip.upload(x), hip.allocate(16)
    # zero columns -> zero outputs; zero rows -> no-op
    hip.copy_to_device(np.full(4, 7.0, np.float32), hy)
    hip.quantized_matmul(hw, hx, hy, 4, 0, dt)
    assert np.all(hip.download(hy, 4) == 0.0)
    hip.quantized_matmul(hw, hx, hy, 0, 256, dt)
    with pytest.raises(YuleGpuError) as e:
        hip.quantized_matmul(hw, hx, hy, 4, 256, 3)   # Q4_1: not on the GPU path
    assert e.value.code == 2
    with pytest.raises(YuleGpuError):
        hip.quantized_matmul(hw, hx, hy, 4, 257, dt)  # needs ceil(257/256) = 2 blocks per row
    with pytest.raises(YuleGpuError):
        hip.quantized_matmul(hw, hx, hy, 5, 256, dt)  # weights too small
    with pytest.raises(YuleGpuError):
        hip.quantized_matmul(hw, hx, hx, 1, 256, dt)  # input aliases output
    with pytest.raises(YuleGpuError):
        hip.quantized_matmul(hw, hx, hw, 1, 256, dt)  # weights alias the output
    with pytest.raises(YuleGpuError):
        hip.quantized_matmul(hw, hw, hy, 1, 256, dt)  # weights alias the input
    with pytest.raises(YuleGpuError):
        hip.quantized_matmul(hw, hx, 999999, 4, 256, dt)  # unknown handle
    for h in (hw, hx, hy):
        hip.free(h)


@pytest.mark.parametrize("dt", FMTS, ids=lambda d: d.name)
@pytest.mark.parametrize("n_rows,n_cols", [(5, 1), (33, 100), (300, 1000), (7, 4097), (64, 14300)])
def test_qmv_ragged_columns(hip, dt, n_rows, n_cols):
    """n_cols not a block multiple: ceil(n_cols/bs) blocks per row with the
    columns >= n_cols skipped (the reference's GPU kernels, cuda/mod.rs:
    311-313 and kernels/cuda/qmv_*.cu); the input holds exactly n_cols
    floats.  Reference: f64 over the bit-exact dequantized rows, first
    n_cols columns."""
    bs = block_size(dt)
    n_pad = -(-n_cols // bs) * bs
    say(f"[qmv] ragged {dt.name} {n_rows}x{n_cols} ({n_pad // bs} blocks per row)")
    w = synth.gen_quant(dt, 400 + n_cols, n_rows, n_pad)
    x = synth.gauss(401, n_cols)
    W = oracle.dequant(int(dt), w).reshape(n_rows, n_pad)[:, :n_cols].astype(np.float64)
    want = W @ x.astype(np.float64)
    hw, hx, hy = hip.upload(w), hip.upload(x), hip.allocate(4 * n_rows)
    hip.quantized_matmul(hw, hx, hy, n_rows, n_cols, dt)
    got = hip.download(hy, n_rows)
    assert np.max(np.abs(got - want)) <= tolerance_bar(want)
    outs = [hip.allocate(4 * n_rows) for _ in range(2)]
    hw2 = hip.upload(w)
    hip.quantized_matmul_multi([hw, hw2], hx, outs, [n_rows, n_rows], n_cols, dt)
    for o in outs:
        assert np.array_equal(hip.download(o, n_rows), got)
    for h in [hw, hw2, hx, hy] + outs:
        hip.free(h)


@pytest.mark.parametrize("dt", FMTS, ids=lambda d: d.name)
def test_qmv_multi_equals_separate_calls(hip, dt):
    """quantized_matmul_multi (Q/K/V- and gate/up-style fusion) returns exactly
    what separate quantized_matmul calls return, for 1..4 matrices."""
    n_cols = 2048
    rows = [2048, 256, 256, 777]
    say(f"[qmv_multi] {dt.name} rows={rows}")
    ws = [synth.gen_quant(dt, 300 + i, r, n_cols) for i, r in enumerate(rows)]
    x = synth.gauss(301, n_cols)
    hx = hip.upload(x)
    hws = [hip.upload(w) for w in ws]
    for n in (1, 2, 3, 4):
        outs = [hip.allocate(4 * r) for r in rows[:n]]
        hip.quantized_matmul_multi(hws[:n], hx, outs, rows[:n], n_cols, dt)
        got = [hip.download(o, r) for o, r in zip(outs, rows)]
        for i in range(n):
            sep = gpu_qmv(hip, dt, ws[i], x, rows[i], n_cols)
            assert np.array_equal(got[i], sep)
            ref = oracle.qmv_f64(int(dt), ws[i], x, rows[i], n_cols)
            assert np.max(np.abs(got[i] - ref)) <= tolerance_bar(ref)
        for o in outs:
            hip.free(o)
    o1, o2 = hip.allocate(4 * 2048), hip.allocate(4 * 256)
    with pytest.raises(YuleGpuError):
        hip.quantized_matmul_multi(hws[:2], hx, [o1, o1], rows[:2], n_cols, dt)   # outputs alias
    with pytest.raises(YuleGpuError):
        hip.quantized_matmul_multi(hws[:2], hx, [o1, hx], rows[:2], n_cols, dt)   # output aliases input
    for h in hws + [hx, o1, o2]:
        hip.free(h)


def test_workspace_users_from_two_threads(hip):
    """Entry points that stage through the backend workspace (ragged
    quantized_matmul, split-KV attention) called concurrently from two host
    threads on one backend: every result equals the single-threaded one."""
    import threading
    say("[qmv] workspace users from two threads")
    jobs = []
    for t in range(2):
        n_rows, n_cols = 300 + 7 * t, 1000 + 13 * t
        dt = DType.Q4_K if t == 0 else DType.Q8_0
        bs = block_size(dt)
        w = synth.gen_quant(dt, 500 + t, n_rows, -(-n_cols // bs) * bs)
        x = synth.gauss(501 + t, n_cols)
        jobs.append((dt, hip.upload(w), hip.upload(x), hip.allocate(4 * n_rows), n_rows, n_cols))
    want = []
    for dt, hw, hx, hy, r, c in jobs:
        hip.quantized_matmul(hw, hx, hy, r, c, dt)
        want.append(hip.download(hy, r))
    nh, nkv, hd, seq = 32, 4, 64, 3000
    q, kc, vc = synth.gauss(8, nh * hd), synth.gauss(9, (seq, nkv * hd)), synth.gauss(10, (seq, nkv * hd))
    hq, hk, hv = hip.upload(q), hip.upload(kc), hip.upload(vc)
    ho = [hip.allocate(4 * nh * hd) for _ in range(2)]
    hip.gqa_decode_attn(hq, hk, hv, ho[0], nh, nkv, hd, seq)
    attn_want = hip.download(ho[0], nh * hd)
    errors = []

    def worker(t):
        try:
            dt, hw, hx, hy, r, c = jobs[t]
            for _ in range(50):
                hip.quantized_matmul(hw, hx, hy, r, c, dt)
                hip.gqa_decode_attn(hq, hk, hv, ho[t], nh, nkv, hd, seq)
        except Exception as e:   # noqa: BLE001
            errors.append(e)
    ths = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for th in ths:
        th.start()
    for th in ths:
        th.join()
    assert not errors
    hip.synchronize()
    for (dt, hw, hx, hy, r, c), wv in zip(jobs, want):
        assert np.array_equal(hip.download(hy, r), wv)
    for h in ho:
        assert np.array_equal(hip.download(h, nh * hd), attn_want)
    for dt, hw, hx, hy, r, c in jobs:
        for h in (hw, hx, hy):
            hip.free(h)
    for h in [hq, hk, hv] + ho:
        hip.free(h)
