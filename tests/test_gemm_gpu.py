"""Prefill dequant-GEMM (yule_hip_quantized_gemm, Q4_0 / Q4_K / Q5_K / Q6_K / Q8_0 / Q8_K) on
the MFMA units: each row
of Y must equal the quantized matvec of the same row of X to the matvec bar
(max|y - y_ref| <= 1e-3 * ||y_ref||_2 / sqrt(N), y_ref the f64 dot of the
bit-exact dequantized weights with the bf16 row converted exactly to f32)."""
import sys

import numpy as np
import pytest

import oracle
from refgen import tolerance_bar
from yule_amd import DType, synth
from yule_amd.backend import YuleGpuError

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 (round to nearest even) as uint16."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def run_gemm(hip, dt, w, xb, M, N, K):
    hw, hx, hy = hip.upload(w), hip.upload(xb), hip.allocate(4 * M * N)
    hip.quantized_gemm(hw, hx, hy, M, N, K, dt)
    y = hip.download(hy, (M, N))
    for h in (hw, hx, hy):
        hip.free(h)
    return y


@pytest.mark.parametrize("dt", [DType.Q4_K, DType.Q6_K, DType.Q8_0, DType.Q4_0, DType.Q5_K, DType.Q8_K],
                         ids=lambda d: d.name)
@pytest.mark.parametrize("M,N,K", [(1, 128, 256), (7, 300, 512), (64, 256, 1024), (130, 129, 2048), (65, 200, 5632)])
def test_gemm_rows_match_oracle(hip, dt, M, N, K):
    say(f"[gemm] {dt.name} M={M} N={N} K={K}")
    w = synth.gen_quant(dt, 50 + M, N, K)
    xb = bf16_bits(synth.gauss(60 + K, (M, K)))
    y = run_gemm(hip, dt, w, xb, M, N, K)
    xf = bf16_to_f32(xb).reshape(M, K)
    for m in range(M):
        ref = oracle.qmv_f64(int(dt), w, xf[m], N, K)
        assert np.max(np.abs(y[m] - ref)) <= tolerance_bar(ref), f"row {m}"


@pytest.mark.parametrize("M", [64, 512])
@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336)])
def test_gemm_config_shapes(hip, N, K, M):
    """BASELINE configs[3] shapes at M = 64 and 512, sampled rows vs the
    oracle; every seventh row against the GPU matvec of the same row."""
    dt = DType.Q4_K
    say(f"[gemm] Q4_K {N}x{K} M={M}")
    w = synth.gen_quant(dt, 70, N, K)
    xb = bf16_bits(synth.gauss(71, (M, K)))
    y = run_gemm(hip, dt, w, xb, M, N, K)
    xf = bf16_to_f32(xb).reshape(M, K)
    for m in (0, 17, 63, M - 1):
        ref = oracle.qmv_f64(int(dt), w, xf[m], N, K)
        assert np.max(np.abs(y[m] - ref)) <= tolerance_bar(ref), f"row {m}"
    hw, hx, hy = hip.upload(w), hip.allocate(4 * K), hip.allocate(4 * N)
    for m in range(0, M, 7):
        hip.copy_to_device(xf[m], hx)
        hip.quantized_matmul(hw, hx, hy, N, K, dt)
        mv = hip.download(hy, N)
        assert np.max(np.abs(y[m] - mv)) <= 2 * tolerance_bar(mv), f"row {m} vs matvec"
    for h in (hw, hx, hy):
        hip.free(h)


@pytest.mark.parametrize("dt,M,N,K", [(DType.Q4_K, 1024, 300, 1024), (DType.Q4_K, 1100, 513, 512),
                                      (DType.Q6_K, 512, 260, 768), (DType.Q6_K, 1030, 129, 256),
                                      (DType.Q8_0, 1024, 300, 1024), (DType.Q4_0, 1100, 513, 512),
                                      (DType.Q5_K, 1024, 300, 1024), (DType.Q8_K, 1030, 129, 512)],
                         ids=lambda v: getattr(v, "name", str(v)))
def test_gemm_wide_tiles(hip, dt, M, N, K):
    """M large enough for the 128 x 256 tiles (eight waves), ragged N and M:
    sampled rows vs the oracle, every row vs the GPU matvec of that row."""
    say(f"[gemm] wide tiles {dt.name} M={M} N={N} K={K}")
    w = synth.gen_quant(dt, 90 + M, N, K)
    xb = bf16_bits(synth.gauss(91 + K, (M, K)))
    y = run_gemm(hip, dt, w, xb, M, N, K)
    xf = bf16_to_f32(xb).reshape(M, K)
    for m in (0, 1, 127, 128, 255, M // 2, M - 1):
        ref = oracle.qmv_f64(int(dt), w, xf[m], N, K)
        assert np.max(np.abs(y[m] - ref)) <= tolerance_bar(ref), f"row {m}"
    hw, hx, hy = hip.upload(w), hip.allocate(4 * K), hip.allocate(4 * N)
    for m in range(M):
        hip.copy_to_device(xf[m], hx)
        hip.quantized_matmul(hw, hx, hy, N, K, dt)
        mv = hip.download(hy, N)
        assert np.max(np.abs(y[m] - mv)) <= 2 * tolerance_bar(mv), f"row {m} vs matvec"
    for h in (hw, hx, hy):
        hip.free(h)


@pytest.mark.parametrize("M,N,K", [(1, 77, 1024), (5, 300, 3072), (16, 64, 2048), (17, 129, 1024),
                                   (32, 200, 3072), (32, 1000, 2048), (8, 4096, 5120), (3, 2000, 14336),
                                   (33, 1000, 2048)])
def test_gemm_few_rows(hip, M, N, K):
    """Q4_K, M <= 32 and K / 256 a multiple of 4: the streaming kernel for
    few X rows (one or two 16-row X tiles; ragged N and M; K splits of one,
    two, five and fourteen super-block groups), every row vs the oracle;
    M = 33 is the tile kernel's again."""
    dt = DType.Q4_K
    say(f"[gemm] few rows Q4_K M={M} N={N} K={K}")
    w = synth.gen_quant(dt, 110 + M, N, K)
    xb = bf16_bits(synth.gauss(111 + K, (M, K)))
    y = run_gemm(hip, dt, w, xb, M, N, K)
    xf = bf16_to_f32(xb).reshape(M, K)
    for m in range(M):
        ref = oracle.qmv_f64(int(dt), w, xf[m], N, K)
        assert np.max(np.abs(y[m] - ref)) <= tolerance_bar(ref), f"row {m}"


@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336)])
def test_gemm_config_shapes_m2048(hip, N, K):
    """BASELINE configs[3] at M=2048, on the 256 x 256 tiles (128 x 64 per
    wave, accumulators rescaled per super-block): 14336x4096 is 448 tiles,
    4096x14336 128 tiles in two K splits.  Rows at tile edges and in the
    last tiles vs the oracle, and a repeat call bit-identical."""
    dt, M = DType.Q4_K, 2048
    say(f"[gemm] Q4_K {N}x{K} M={M}")
    w = synth.gen_quant(dt, 72, N, K)
    xb = bf16_bits(synth.gauss(73, (M, K)))
    y = run_gemm(hip, dt, w, xb, M, N, K)
    assert np.array_equal(y, run_gemm(hip, dt, w, xb, M, N, K)), "second call differs"
    xf = bf16_to_f32(xb).reshape(M, K)
    for m in (0, 255, 256, 1663, 1664, 1800, 2047):
        ref = oracle.qmv_f64(int(dt), w, xf[m], N, K)
        assert np.max(np.abs(y[m] - ref)) <= tolerance_bar(ref), f"row {m}"


# Shapes whose tile count passes a whole round of resident workgroups (256
# CUs: one 128 x 256 tile or two 128 x 128 tiles per CU) by at most half a
# round: the last tiles then run as two K halves added into zeroed y.  The
# last two cases take the 64-row tiles (M <= 64) with lm_head-like widths.
@pytest.mark.parametrize("dt,M,N,K", [(DType.Q4_K, 1024, 8348, 512), (DType.Q4_K, 1100, 7673, 768),
                                      (DType.Q5_K, 1024, 8348, 512), (DType.Q6_K, 512, 16590, 512),
                                      (DType.Q8_0, 512, 16512, 512), (DType.Q4_0, 1024, 8348, 512),
                                      (DType.Q8_K, 1024, 8348, 512), (DType.Q4_K, 40, 66000, 512),
                                      (DType.Q6_K, 64, 65800, 768)],
                         ids=lambda v: getattr(v, "name", str(v)))
def test_gemm_tail_halves(hip, dt, M, N, K):
    """The last m tiles (where the split tail tiles lie) vs the oracle, every
    row vs the GPU matvec, and a second call bit-identical to the first."""
    say(f"[gemm] tail halves {dt.name} M={M} N={N} K={K}")
    w = synth.gen_quant(dt, 70 + M, N, K)
    xb = bf16_bits(synth.gauss(71 + K, (M, K)))
    y = run_gemm(hip, dt, w, xb, M, N, K)
    assert np.array_equal(y, run_gemm(hip, dt, w, xb, M, N, K)), "second call differs"
    xf = bf16_to_f32(xb).reshape(M, K)
    for m in sorted({0, max(M - 129, 0), max(M - 128, 0), max(M - 65, 0), M - 2, M - 1}):
        ref = oracle.qmv_f64(int(dt), w, xf[m], N, K)
        assert np.max(np.abs(y[m] - ref)) <= tolerance_bar(ref), f"row {m}"
    hw, hx, hy = hip.upload(w), hip.allocate(4 * K), hip.allocate(4 * N)
    for m in range(M):
        hip.copy_to_device(xf[m], hx)
        hip.quantized_matmul(hw, hx, hy, N, K, dt)
        mv = hip.download(hy, N)
        assert np.max(np.abs(y[m] - mv)) <= 2 * tolerance_bar(mv), f"row {m} vs matvec"
    for h in (hw, hx, hy):
        hip.free(h)


ALL_GEMM = [DType.Q4_K, DType.Q6_K, DType.Q8_0, DType.Q4_0, DType.Q5_K, DType.Q8_K]


def range_rows(K: int) -> np.ndarray:
    """Rows that leave f16's range or precision unscaled: magnitudes 1e5 and
    1e36, 1e-7 and 1e-30, a row of 2100s (sub-block sums of 67200 > 65504),
    a row of small values holding two 3e38 elements, zeros, and N(0,1)."""
    g = np.random.default_rng(K)
    n = lambda: g.standard_normal(K)
    big = 1e-3 * n()
    big[[5, K - 7]] = 3e38
    rows = [1e5 * n(), 1e36 * n(), 1e-7 * n(), 1e-30 * n(), np.full(K, 2100.0), big, np.zeros(K), n()]
    return np.array(rows, np.float32)


@pytest.mark.parametrize("dt", ALL_GEMM, ids=lambda d: d.name)
@pytest.mark.parametrize("M", [8, 136])
def test_gemm_bf16_full_range(hip, dt, M):
    """Any finite bf16 row: each row against the oracle's f64 dot of the same
    bf16-valued row (the per-row power-of-two scale is exact)."""
    N, K = 160, 1024
    say(f"[gemm] bf16 range rows {dt.name} M={M}")
    w = synth.gen_quant(dt, 95, N, K)
    base = range_rows(K)
    xb = bf16_bits(np.concatenate([base] * (M // len(base)) + [base[:M % len(base)]]))
    y = run_gemm(hip, dt, w, xb, M, N, K)
    xf = bf16_to_f32(xb).reshape(M, K)
    for m in range(M):
        ref = oracle.qmv_f64(int(dt), w, xf[m], N, K)
        if not np.any(xf[m]):
            assert np.all(y[m] == 0.0), f"row {m}"
            continue
        assert np.all(np.isfinite(y[m])), f"row {m}"
        assert np.max(np.abs(y[m] - ref)) <= tolerance_bar(ref), f"row {m}"


def run_gemm_f32(hip, dt, w, x, M, N, K):
    hw, hx, hy = hip.upload(w), hip.upload(np.ascontiguousarray(x, np.float32)), hip.allocate(4 * M * N)
    hip.quantized_gemm_f32(hw, hx, hy, M, N, K, dt)
    y = hip.download(hy, (M, N))
    for h in (hw, hx, hy):
        hip.free(h)
    return y


@pytest.mark.parametrize("dt", ALL_GEMM, ids=lambda d: d.name)
@pytest.mark.parametrize("M,N,K", [(1, 128, 256), (7, 300, 512), (128, 2560, 2048), (128, 2048, 5632),
                                   (130, 129, 2048), (1024, 300, 1024)])
def test_gemm_f32_rows_match_oracle(hip, dt, M, N, K):
    """f32 X (hi + lo on the matrix cores): rows against the oracle's f64 dot
    of the same f32 row, and against the GPU's f32 matvec of that row."""
    say(f"[gemm f32] {dt.name} M={M} N={N} K={K}")
    w = synth.gen_quant(dt, 110 + M, N, K)
    x = synth.gauss(111 + K, (M, K))
    y = run_gemm_f32(hip, dt, w, x, M, N, K)
    rows = sorted({0, M // 2, M - 1} | set(range(0, M, max(1, M // 8))))
    for m in rows:
        ref = oracle.qmv_f64(int(dt), w, x[m], N, K)
        assert np.max(np.abs(y[m] - ref)) <= tolerance_bar(ref), f"row {m}"
    hw, hx, hy = hip.upload(w), hip.allocate(4 * K), hip.allocate(4 * N)
    for m in rows:
        hip.copy_to_device(x[m], hx)
        hip.quantized_matmul(hw, hx, hy, N, K, dt)
        mv = hip.download(hy, N)
        assert np.max(np.abs(y[m] - mv)) <= tolerance_bar(mv), f"row {m} vs matvec"
    for h in (hw, hx, hy):
        hip.free(h)


@pytest.mark.parametrize("dt", [DType.Q4_K, DType.Q6_K, DType.Q8_0], ids=lambda d: d.name)
def test_gemm_f32_full_range_and_repeat(hip, dt):
    """f32 rows of any magnitude, and a second call bit-identical (the lo
    product adds into Y in a fixed order: split-K at M = 16, whole tiles at
    M = 1024 where the bf16 call would split its tail tiles)."""
    K = 1024
    say(f"[gemm f32] range rows and repeat {dt.name}")
    w = synth.gen_quant(dt, 120, 160, K)
    x = range_rows(K)
    y = run_gemm_f32(hip, dt, w, x, len(x), 160, K)
    for m in range(len(x)):
        ref = oracle.qmv_f64(int(dt), w, x[m], 160, K)
        if not np.any(x[m]):
            assert np.all(y[m] == 0.0)
            continue
        assert np.all(np.isfinite(y[m])) and np.max(np.abs(y[m] - ref)) <= tolerance_bar(ref), f"row {m}"
    for M, N, KK in ((16, 4096, 4096), (1024, 8348, 512)):
        w2 = synth.gen_quant(dt, 121, N, KK)
        x2 = synth.gauss(122, (M, KK))
        a = run_gemm_f32(hip, dt, w2, x2, M, N, KK)
        assert np.array_equal(a, run_gemm_f32(hip, dt, w2, x2, M, N, KK)), f"M={M}: second call differs"
        ref = oracle.qmv_f64(int(dt), w2, x2[M - 1], N, KK)
        assert np.max(np.abs(a[M - 1] - ref)) <= tolerance_bar(ref)


def test_gemm_errors(hip):
    w = synth.gen_quant(DType.Q4_K, 1, 16, 256)
    hw, hx, hy = hip.upload(w), hip.allocate(2 * 256 * 4), hip.allocate(4 * 16 * 4)
    with pytest.raises(YuleGpuError):
        hip.quantized_gemm(hw, hx, hy, 4, 16, 256, DType.F16)       # not on the MFMA path
    with pytest.raises(YuleGpuError):
        hip.quantized_gemm(hw, hx, hy, 5, 16, 256, DType.Q4_K)      # x too small
    with pytest.raises(YuleGpuError):
        hip.quantized_gemm(hw, hx, hx, 1, 16, 256, DType.Q4_K)      # x aliases y
    with pytest.raises(YuleGpuError):
        hip.quantized_gemm(hw, hx, hw, 1, 16, 256, DType.Q4_K)      # weights alias y
    with pytest.raises(YuleGpuError):
        hip.quantized_gemm(hw, hw, hy, 1, 16, 256, DType.Q4_K)      # weights alias x
    for h in (hw, hx, hy):
        hip.free(h)
