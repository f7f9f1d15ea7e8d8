"""yule_hip_quantized_gemm_noalloc (static per-GPU workspace, no allocation)
against yule_hip_quantized_gemm through the C ABI: two calls in a row, the
second smaller and in another format, must give the same Y (same kernels,
so bit-identical, which is within the matvec bar); a call whose workspace
would exceed the static array is refused."""
import sys

import numpy as np
import pytest

import oracle
from refgen import tolerance_bar
from yule_amd import DType, synth
from yule_amd.backend import YuleGpuError

pytestmark = pytest.mark.gpu


def bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def both(hip, dt, M, N, K, seed):
    w = synth.gen_quant(dt, seed, N, K)
    xb = bf16_bits(synth.gauss(seed + 1, (M, K)))
    hw, hx, hy, hz = hip.upload(w), hip.upload(xb), hip.allocate(4 * M * N), hip.allocate(4 * M * N)
    hip.quantized_gemm_noalloc(hw, hx, hy, M, N, K, dt)
    hip.quantized_gemm(hw, hx, hz, M, N, K, dt)
    y, z = hip.download(hy, (M, N)), hip.download(hz, (M, N))
    for h in (hw, hx, hy, hz):
        hip.free(h)
    return w, xb, y, z


def test_noalloc_gemm_matches_allocating_entry(hip):
    print("[noalloc] Q4_K 128x2560x2048, then Q6_K 16x1024x1024 (split-K)", flush=True)
    for dt, M, N, K, seed in ((DType.Q4_K, 128, 2560, 2048, 131), (DType.Q6_K, 16, 1024, 1024, 133)):
        w, xb, y, z = both(hip, dt, M, N, K, seed)
        assert np.array_equal(y, z), f"{dt.name} M={M}: differs from quantized_gemm"
        xf = (xb.astype(np.uint32) << 16).view(np.float32).reshape(M, K)
        for m in (0, M - 1):
            ref = oracle.qmv_f64(int(dt), w, xf[m], N, K)
            assert np.max(np.abs(y[m] - ref)) <= tolerance_bar(ref)


def test_noalloc_gemm_refuses_oversize(hip):
    M, N, K = 2048, 256, 14336   # X alone is 58.7 MB of f16
    hw, hx, hy = hip.allocate(N * (K // 256) * 144), hip.allocate(2 * M * K), hip.allocate(4 * M * N)
    with pytest.raises(YuleGpuError, match="static"):
        hip.quantized_gemm_noalloc(hw, hx, hy, M, N, K, DType.Q4_K)
    for h in (hw, hx, hy):
        hip.free(h)


def test_noalloc_gemm_under_graph_capture(hip):
    """The allocation-free entry enqueues cleanly under HIP stream capture
    (one single-split and one split-K shape in one graph); every replay,
    with eager work and host synchronizations between replays, gives the
    allocating entry's Y bit for bit."""
    print("[noalloc] graph capture: Q4_K 128x2560x2048 and Q6_K 16x1024x1024", flush=True)
    cases = []
    for dt, M, N, K, seed in ((DType.Q4_K, 128, 2560, 2048, 141), (DType.Q6_K, 16, 1024, 1024, 143)):
        w = synth.gen_quant(dt, seed, N, K)
        xb = bf16_bits(synth.gauss(seed + 1, (M, K)))
        hw, hx, hy, hz = hip.upload(w), hip.upload(xb), hip.allocate(4 * M * N), hip.allocate(4 * M * N)
        hip.quantized_gemm(hw, hx, hz, M, N, K, dt)
        cases.append((dt, M, N, K, hw, hx, hy, hip.download(hz, (M, N)), hz))
    hip.synchronize()
    hip.capture_begin()
    try:
        for dt, M, N, K, hw, hx, hy, _, _ in cases:
            hip.quantized_gemm_noalloc(hw, hx, hy, M, N, K, dt)
    finally:
        hip.capture_end()
    for rep in range(3):
        for dt, M, N, K, hw, hx, hy, want, hz in cases:
            hip.copy_to_device(np.full(M * N, np.nan, np.float32), hy)   # stale Y must not survive
            hip.quantized_gemm(hw, hx, hz, M, N, K, dt)                  # eager work between replays
        hip.capture_replay()
        hip.synchronize()
        for dt, M, N, K, hw, hx, hy, want, hz in cases:
            assert np.array_equal(hip.download(hy, (M, N)), want), f"replay {rep}: {dt.name} M={M} differs"
    for c in cases:
        for h in (c[4], c[5], c[6], c[8]):
            hip.free(h)
