"""bench.py — Q4_K decode matvec throughput on one MI355X (BASELINE metric).

A "step" is one pass of the hot path over one batch of synthetic input: the
seven batch-1 projections of one Llama-3-8B layer (Q 4096x4096, K and V
1024x4096, O 4096x4096, gate and up 14336x4096, down 4096x14336) in Q4_K
over raw GGUF blocks, launched as the HIP runner
launches them: Q/K/V in one `quantized_matmul_multi` (they share the normed
input), O, gate/up in one, down.  The same layer as seven separate
`quantized_matmul` calls is reported beside it.
Steps cycle through `--copies` distinct copies of the layer (8 x 122.7 MB by
default) so no step re-reads weights left in the 256 MB last-level cache;
all inputs are resident in HBM before the timed region.  Timing: HIP events
recorded on the backend stream around a HIP graph holding exactly K steps,
bracketed by device synchronisation.

value = algorithmic bytes of K steps (weights + x + y of every projection)
/ elapsed seconds, in GB/s.  Extra fields report the per-matrix rates, the
Q6_K/Q8_0 layers, the TinyLlama-shape sweep, the roofline of
the dominant kernel (Q4_K 14336x4096) and the CPU baseline: the oracle's
restatement of Yule's AVX2 qmv (oracle/cpu_avx2.c) timed on the host cores.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--copies C] [--quick]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from yule_amd import DType, matrix_bytes, synth  # noqa: E402

METRIC = "Q4_K matvec HBM GB/s (% of 8 TB/s peak); Q4_K_M decode tokens/sec, 1 GPU"
HBM_PEAK_GBS = 8000.0

# Llama-3-8B per-layer projections (n_rows, n_cols)
LLAMA3_LAYER = [("attn_q", 4096, 4096), ("attn_k", 1024, 4096), ("attn_v", 1024, 4096),
                ("attn_output", 4096, 4096), ("ffn_gate", 14336, 4096), ("ffn_up", 14336, 4096),
                ("ffn_down", 4096, 14336)]
LLAMA3_LM_HEAD = ("output", 128256, 4096)
# TinyLlama-1.1B projections
# TinyLlama-1.1B layer projections (the runner's decode launches, configs[1]'s Q4_K shapes)
TINY_LAYER = [("attn_q", 2048, 2048), ("attn_k", 256, 2048), ("attn_v", 256, 2048), ("attn_output", 2048, 2048),
              ("ffn_gate", 5632, 2048), ("ffn_up", 5632, 2048), ("ffn_down", 2048, 5632)]
TINY_SWEEP = [("q_o", 2048, 2048, DType.Q4_K), ("k_v", 256, 2048, DType.Q4_K), ("gate_up", 5632, 2048, DType.Q4_K),
              ("down", 2048, 5632, DType.Q4_K), ("lm_head", 32000, 2048, DType.Q6_K)]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def algo_bytes(dt, n_rows, n_cols) -> int:
    """Algorithmic bytes of one matvec: the weight blocks + f32 x + f32 y."""
    return matrix_bytes(dt, n_rows, n_cols) + 4 * n_cols + 4 * n_rows


class Layer:
    """`copies` device copies of one layer's projections in one format."""

    def __init__(self, hip, dt, shapes, copies, seed):
        self.hip, self.dt, self.shapes = hip, dt, shapes
        self.host = {}
        self.w = {}
        self.x = {}
        self.y = {}
        for i, (name, r, c) in enumerate(shapes):
            t0 = time.time()
            self.host[name] = synth.gen_quant(dt, seed + i, r, c)
            self.w[name] = [hip.upload(self.host[name]) for _ in range(copies)]
            if c not in self.x:
                xs = synth.gauss(seed + 1000 + c, c)
                self.host[f"x{c}"] = xs
                self.x[c] = hip.upload(xs)
            self.y[name] = [hip.allocate(4 * r) for _ in range(copies)]
            log(f"  {dt.name} {name} {r}x{c}: {matrix_bytes(dt, r, c) / 1e6:.1f} MB x{copies} ({time.time() - t0:.1f}s)")
        self.copies = copies
        self.step_bytes = sum(algo_bytes(dt, r, c) for _, r, c in shapes)

    def ops_for_step(self, s, fused=True):
        """One layer pass.  fused: the HIP runner's launches -- Q/K/V as one
        multi-matrix launch, O, gate/up as one, down; else seven calls."""
        c = s % self.copies
        if not fused or [n for n, _, _ in self.shapes] != [n for n, _, _ in LLAMA3_LAYER]:   # names, not sizes
            return [(self.w[n][c], self.x[cols], self.y[n][c], r, cols, self.dt) for n, r, cols in self.shapes]
        sh = {n: (r, cols) for n, r, cols in self.shapes}

        def group(names):
            cols = sh[names[0]][1]
            return ([self.w[n][c] for n in names], self.x[cols], [self.y[n][c] for n in names],
                    [sh[n][0] for n in names], cols, self.dt)
        return [group(["attn_q", "attn_k", "attn_v"]), group(["attn_output"]), group(["ffn_gate", "ffn_up"]),
                group(["ffn_down"])]

    def ops_for_matrix(self, name, n):
        _, r, cols = next(s for s in self.shapes if s[0] == name)
        return [(self.w[name][i % self.copies], self.x[cols], self.y[name][i % self.copies], r, cols, self.dt)
                for i in range(n)]

    def free(self):
        for lst in list(self.w.values()) + list(self.y.values()):
            for h in lst:
                self.hip.free(h)
        for h in self.x.values():
            self.hip.free(h)


USE_GRAPH = True
DOM_COPIES = 32   # copies of the dominant matrix cycled by its roofline measurement


def time_steps(hip, layer, steps, start=0, fused=True):
    ops = [op for s in range(start, start + steps) for op in layer.ops_for_step(s, fused)]
    hip.synchronize()
    ms = hip.time_qmv_ops(ops, 1, use_graph=USE_GRAPH)
    hip.synchronize()
    return ms


def matrix_rate(hip, layer, name, launches):
    _, r, c = next(s for s in layer.shapes if s[0] == name)
    hip.time_qmv_ops(layer.ops_for_matrix(name, min(launches, 64)), 1, USE_GRAPH)       # warm-up
    ms = hip.time_qmv_ops(layer.ops_for_matrix(name, launches), 1, USE_GRAPH)
    us = 1e3 * ms / launches
    gbs = algo_bytes(layer.dt, r, c) / (us * 1e-6) / 1e9
    return us, gbs


def read_probe(hip, layer, name, launches, n_wg=2048, pattern=None, loads=1):
    """What one launch that only streams the same weight bytes achieves, over
    the same rotating copies as the matrix it stands beside: yule_hip_read_probe
    (grid-stride 16-byte loads) or, with `pattern`, yule_hip_read_probe_variant.
    The XOR checksum of the first launch is checked against the host bytes;
    the median of 5 timed passes is reported."""
    _, r, c = next(s for s in layer.shapes if s[0] == name)
    nbytes = matrix_bytes(layer.dt, r, c)
    part = hip.allocate(4 * n_wg)

    def go(w):
        if pattern is None:
            hip.read_probe(w, nbytes, part, n_wg)
        else:
            hip.read_probe_variant(w, nbytes, part, n_wg, pattern, loads)
    go(layer.w[name][0])
    got = int(np.bitwise_xor.reduce(hip.download(part, n_wg, np.uint32)))
    want = int(np.bitwise_xor.reduce(np.ascontiguousarray(layer.host[name]).view(np.uint32).ravel()))
    if got != want:
        raise RuntimeError(f"read probe checksum {got:#x} != host {want:#x}")
    for i in range(64):
        go(layer.w[name][i % layer.copies])
    runs = []
    for _ in range(5):
        hip.timer_start()
        for i in range(launches):
            go(layer.w[name][i % layer.copies])
        runs.append(hip.timer_stop() * 1e3 / launches)
    us = float(np.median(runs))
    hip.free(part)
    what = ("yule_hip_read_probe (grid-stride 16-byte words)" if pattern is None else
            f"yule_hip_read_probe_variant pattern {pattern}, {loads} words per lane")
    return {"us": round(us, 3), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1), "bytes": nbytes,
            "launch": f"{what}, {n_wg} x 256 threads, back-to-back stream launches, median of 5 passes"}


def dominant_rate(hip, dom, launches=1000, passes=5):
    """Average launch duration of the dominant matvec (Q4_K 14336x4096): HIP
    events around `launches` back-to-back launches replayed from one graph,
    cycling the layer's weight copies; median over `passes` timed passes after
    one warm-up pass."""
    _, r, c = dom.shapes[0]
    ops = dom.ops_for_matrix("ffn_gate", launches)
    hip.time_qmv_ops(ops[:64], 1, USE_GRAPH)
    runs = sorted(1e3 * hip.time_qmv_ops(ops, 1, USE_GRAPH) / launches for _ in range(passes))
    us = runs[len(runs) // 2]
    return us, algo_bytes(dom.dt, r, c) / (us * 1e-6) / 1e9, runs


def _time_qmv_layer(layer, threads, budget_s, max_passes):
    import oracle
    mats = [(layer.host[n], layer.host[f"x{c}"], r, c) for n, r, c in layer.shapes]
    for w, x, r, c in mats:                       # warm-up pass
        oracle.qmv(int(layer.dt), w, x, r, c, threads)
    passes, t0 = 0, time.perf_counter()
    while passes < max_passes and (passes < 2 or time.perf_counter() - t0 < budget_s):
        for w, x, r, c in mats:
            oracle.qmv(int(layer.dt), w, x, r, c, threads)
        passes += 1
    dt = time.perf_counter() - t0
    return passes * layer.step_bytes / dt / 1e9, passes, dt


def cpu_baseline(layer, budget_s=12.0, max_passes=2000):
    """Yule's CPU decode matvec path over the same Q4_K layer bytes,
    host-resident: the oracle's restatement of model_runner.rs:152-244 (the
    per-call std::thread row split).  When oracle/_ref holds the reference's
    own Q4_K assembly kernel (yule-core/src/kernels/q4k_gemv_avx2.S, which
    the reference's AVX2 build uses for every Q4_K block, simd/avx2.rs:
    84-96), the block dots run through it and the baseline is
    kind "reference"; the pure restatement (the Rust-fallback AVX2 body) is
    reported beside it.  Otherwise the restatement alone, kind "port"."""
    import oracle
    threads = min(16, os.cpu_count() or 1)
    asm = oracle.q4k_asm() if layer.dt == DType.Q4_K else None
    if asm is None:
        gbs, passes, dt = _time_qmv_layer(layer, threads, budget_s, max_passes)
        return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
                "sample": f"{passes} passes of the Q4_K Llama-3-8B layer (7 projections, "
                          f"{layer.step_bytes / 1e6:.1f} MB each pass) through the oracle's restatement of Yule's "
                          f"AVX2 qmv with a per-call std::thread row split, {threads} threads, {dt:.1f} s",
                "host_cpu": host_cpu_record(threads)}
    port, _, _ = _time_qmv_layer(layer, threads, budget_s / 2, max_passes)
    oracle.set_q4k_dot(asm)
    try:
        gbs, passes, dt = _time_qmv_layer(layer, threads, budget_s / 2, max_passes)
    finally:
        oracle.set_q4k_dot(None)
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "reference",
            "sample": f"{passes} passes of the Q4_K Llama-3-8B layer (7 projections, "
                      f"{layer.step_bytes / 1e6:.1f} MB each pass): the reference's q4k_gemv_avx2.S (assembled from "
                      f"its sources into oracle/_ref) for every block, inside the restatement of model_runner.rs "
                      f"qmv's per-call std::thread row split, {threads} threads, {dt:.1f} s",
            "port_value": round(port, 3), "host_cpu": host_cpu_record(threads)}


def decode_e2e(hip, cpu: bool, cpu_steps: int = 256):
    """TinyLlama-shaped Q4_K_M greedy decode, 128-token
    prompt then 256 decode steps, tok/s = 1000 / mean decode-step ms
    (yule-validate/src/performance.rs:303-337)."""
    from yule_amd.backend import HipRunner
    from yule_amd.model import TINYLLAMA, SyntheticModel
    t0 = time.time()
    model = SyntheticModel.generate(TINYLLAMA, seed=0)
    log(f"TinyLlama-shaped model: {model.weight_bytes / 1e6:.0f} MB ({time.time() - t0:.1f}s)")
    prompt = synth.uniform_tokens(1, 128, TINYLLAMA.vocab)
    run = HipRunner(hip, model)
    run.generate_greedy(prompt, 16)                       # warm-up (graph capture)
    toks, ms = run.generate_greedy(prompt, 256)
    pre_ms = run.last_prefill_ms
    run.close()
    res = {"decode_tok_s": round(1000.0 / ms, 1), "decode_ms_per_step": round(ms, 4),
           # the 128-token prompt as one batched pass (GEMM projections, causal
           # attention per row), prompt tokens / wall ms of that pass
           "prefill_tok_s": round(len(prompt) * 1000.0 / pre_ms, 1), "prefill_ms": round(pre_ms, 3),
           "decode_weight_bytes_per_step": model.bytes_per_token(),
           "decode_effective_GB/s": round(model.bytes_per_token() / (ms * 1e-3) / 1e9, 1)}
    golden = ROOT / "tests" / "golden" / "e2e_tinyllama_greedy.json"
    if golden.exists():
        res["decode_tokens_match_oracle"] = [int(t) for t in toks] == json.loads(golden.read_text())["tokens"]
    if cpu:
        import oracle
        threads = min(16, os.cpu_count() or 1)
        asm = oracle.q4k_asm()          # the reference's Q4_K assembly kernel, as its AVX2 build runs it
        if asm is not None:
            oracle.set_q4k_dot(asm)
        try:
            # the GPU figure's workload: the 128-token prompt (untimed), then
            # all 256 greedy decode steps, positions 128..383
            r = oracle.Runner(model, n_threads=threads)
            t0 = time.perf_counter()
            for t in prompt:
                logits = r.forward(int(t))
            pre_s = time.perf_counter() - t0
            n, t0 = 0, time.perf_counter()
            cpu_toks = [oracle.argmax(logits)]
            while n < cpu_steps:
                logits = r.forward(cpu_toks[-1])
                cpu_toks.append(oracle.argmax(logits))
                n += 1
            cms = 1e3 * (time.perf_counter() - t0) / n
        finally:
            oracle.set_q4k_dot(None)
        what = ("the reference's q4k_gemv_avx2.S for every Q4_K block" if asm is not None
                else "the Rust-fallback restatement of the AVX2 Q4_K body")
        res["cpu_decode"] = {"tok_s": round(1000.0 / cms, 2), "threads": threads,
                             "kind": "reference" if asm is not None else "port",
                             "prompt_tok_s": round(len(prompt) / pre_s, 2),
                             "sample": f"the same 128-token prompt (token by token, untimed in tok_s), then {n} "
                                       f"greedy decode steps at positions 128..{127 + n} (the GPU run decodes "
                                       f"128..383), through the oracle's restatement of Yule's CPU "
                                       f"TransformerRunner with {what}",
                             "tokens_match_gpu": [int(t) for t in cpu_toks] == [int(t) for t in toks[:n + 1]],
                             "host_cpu": host_cpu_record(threads)}
        res["decode_speedup_vs_cpu"] = round(cms / ms, 1)
    return res


MFMA_F16_PEAK_TFLOPS = 2500.0   # MI355X dense f16/bf16 MFMA


def prefill_gemm(hip, dt=DType.Q4_K, shapes=((14336, 4096), (4096, 14336)), ms_=(64, 512, 2048)):
    """Q4_K 14336x4096 and 4096x14336 weights times a bf16
    activation matrix of M in {64, 512, 2048} rows, on the MFMA path (other
    formats: the same kernel family, reported beside it)."""
    out = {}
    for n_rows, n_cols in shapes:
        w = hip.upload(synth.gen_quant(dt, 81, n_rows, n_cols))
        for M in ms_:
            xb = (synth.gauss(82, (M, n_cols)).view(np.uint32) >> 16).astype(np.uint16)   # bf16 (truncated)
            hx, hy = hip.upload(xb), hip.allocate(4 * M * n_rows)
            reps = max(3, min(50, int(2e4 // M)))
            hip.quantized_gemm(w, hx, hy, M, n_rows, n_cols, dt)   # warm-up
            hip.synchronize()
            hip.timer_start()
            for _ in range(reps):
                hip.quantized_gemm(w, hx, hy, M, n_rows, n_cols, dt)
            ms = hip.timer_stop() / reps
            tflops = 2.0 * M * n_rows * n_cols / (ms * 1e-3) / 1e12
            out[f"{n_rows}x{n_cols} M={M}"] = {"us": round(ms * 1e3, 1), "TFLOP/s": round(tflops, 1),
                                               "mfma_util": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)}
            log(f"prefill GEMM {dt.name} {n_rows}x{n_cols} M={M}: {ms * 1e3:.1f} us, {tflops:.1f} TFLOP/s")
            hip.free(hx)
            hip.free(hy)
        hip.free(w)
    return out


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_cpu_record(threads_used: int) -> dict:
    """The host the CPU baseline ran on: model, logical CPUs the process may
    use, physical cores behind them (distinct core ids per package), SMT
    state, and the threads the baseline used."""
    logical = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else list(range(os.cpu_count() or 1))
    cores = set()
    for c in logical:
        try:
            pkg = open(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id").read().strip()
            core = open(f"/sys/devices/system/cpu/cpu{c}/topology/core_id").read().strip()
            cores.add((pkg, core))
        except OSError:
            cores.add(("?", str(c)))
    try:
        smt = open("/sys/devices/system/cpu/smt/active").read().strip() == "1"
    except OSError:
        smt = None
    fam = {}
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k = k.strip()
            if k in ("vendor_id", "cpu family", "model", "stepping") and k not in fam:
                fam[k] = v.strip()
            if not line.strip():
                break
    except OSError:
        pass
    return {"model": _cpu_model(), "cpuid": fam, "logical_cpus_available": len(logical), "physical_cores_available": len(cores),
            "smt_active": smt, "threads_used": threads_used, "machine_logical_cpus": os.cpu_count()}


def dominant_kernel_name():
    """The kernel the library launches for a Q4_K 14336x4096 matvec under the
    current environment (the switches qmv.hip reads: YULE_QMV_V1 selects the
    column-looping kernel, YULE_QMV_THREADS_W64 the workgroup size of one-wave
    teams; non-positive or unparsable values keep the default)."""
    if os.environ.get("YULE_QMV_V1") is not None:
        return "qmv_kernel<Q4K,64,*>"
    try:
        nt = int(os.environ.get("YULE_QMV_THREADS_W64", "512"))
    except ValueError:
        nt = 512
    nt = nt if nt > 0 else 512
    nt = 1024 if nt >= 1024 else 512 if nt >= 512 else 256
    return f"qmv_stream_kernel<Q4K,64,2,{nt}>"


def traffic_from_profiles():
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3
    --pmc summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel factor)."""
    p = ROOT / "profiles" / "qmv_q4k_14336x4096_traffic.json"
    if p.exists():
        try:
            return json.loads(p.read_text()).get("bytes_per_launch")
        except Exception:
            return None
    return None


def profile_avg_us():
    """Average duration of the dominant kernel in the committed rocprofv3
    kernel-trace summary of `bench.py --profile-dominant` (None if absent)."""
    p = ROOT / "profiles" / "qmv_q4k_14336x4096_traffic.json"
    try:
        return json.loads(p.read_text()).get("trace_avg_us")
    except Exception:
        return None


def profile_dominant(hip, n, copies):
    """Dominant-kernel-only run for rocprofv3 (kernel trace, or --pmc counters):
    the bench's own roofline measurement of the Q4_K 14336x4096 matvec (64
    warm-up launches, then 5 passes of N launches replayed from a graph,
    cycling the weight copies), then one 64 MiB buffer copy whose counters
    calibrate the bytes-per-KiB scale of FETCH_SIZE / WRITE_SIZE."""
    L = Layer(hip, DType.Q4_K, [("ffn_gate", 14336, 4096)], max(copies, DOM_COPIES), seed=11)
    us, _, runs = dominant_rate(hip, L, n)    # exactly the bench's roofline measurement
    src, dst = hip.allocate(64 << 20), hip.allocate(64 << 20)
    hip.copy_buffer(src, dst, 64 << 20)
    hip.synchronize()
    print(json.dumps({"launches": n, "us_per_launch": round(us, 3), "passes_us": [round(u, 3) for u in runs],
                      "algo_bytes_per_launch": algo_bytes(DType.Q4_K, 14336, 4096),
                      "calibration_copy_bytes": 64 << 20}), flush=True)


def probe_curve(hip, sizes_mb=(33, 128, 256, 558, 1024), n_wgs=(1024, 2048, 4096, 8192)):
    """Single-launch streaming-read rate against launch size: yule_hip_read_probe
    over rotating buffers totalling >= 2 GiB (beyond the 256 MB last-level
    cache), median of the per-launch rates of 5 timed passes.  Prints one JSON line."""
    out = {}
    for mb in sizes_mb:
        nbytes = (mb * 1000 * 1000) // 4096 * 4096
        copies = max(2, -(-(2 << 30) // nbytes))
        bufs = [hip.allocate(nbytes) for _ in range(copies)]
        row = {}
        for n_wg in n_wgs:
            part = hip.allocate(4 * n_wg)
            launches = max(2 * copies, min(2000, int(4e9 // nbytes)))
            for i in range(copies):
                hip.read_probe(bufs[i], nbytes, part, n_wg)
            rates = []
            for _ in range(5):
                hip.timer_start()
                for i in range(launches):
                    hip.read_probe(bufs[i % copies], nbytes, part, n_wg)
                us = hip.timer_stop() * 1e3 / launches
                rates.append(nbytes / (us * 1e-6) / 1e9)
            hip.free(part)
            g = float(np.median(rates))
            row[str(n_wg)] = {"us": round(nbytes / (g * 1e9) * 1e6, 3), "GB/s": round(g, 1)}
            log(f"read probe {mb} MB, {n_wg} workgroups: {row[str(n_wg)]['us']} us, {g:.1f} GB/s")
        for b in bufs:
            hip.free(b)
        out[f"{mb}MB"] = row
    print(json.dumps({"read_probe_curve": out, "launch": "yule_hip_read_probe, 256-thread workgroups, "
                      "back-to-back stream launches over rotating buffers, HIP events"}), flush=True)


def probe_variants(hip, sizes_mb=(33, 128), grids=(512, 1024, 2048, 4096)):
    """Single-launch streaming-read rate by access pattern (yule_hip_read_probe_variant:
    0 grid-stride words with 1/2/4/8 loads in flight per lane, 1 per-lane runs of
    16-128 bytes, 2 one contiguous chunk per workgroup) and grid size, over rotating
    buffers totalling >= 2 GiB; median of 5 timed passes.  Prints one JSON line."""
    out = {}
    for mb in sizes_mb:
        nbytes = (mb * 1000 * 1000) // 4096 * 4096
        copies = max(2, -(-(2 << 30) // nbytes))
        bufs = [hip.allocate(nbytes) for _ in range(copies)]
        launches = max(2 * copies, min(2000, int(4e9 // nbytes)))
        best = None
        for pattern in (0, 1, 2):
            for loads in (1, 2, 4, 8):
                for n_wg in grids:
                    part = hip.allocate(4 * n_wg)
                    for i in range(copies):
                        hip.read_probe_variant(bufs[i], nbytes, part, n_wg, pattern, loads)
                    rates = []
                    for _ in range(5):
                        hip.timer_start()
                        for i in range(launches):
                            hip.read_probe_variant(bufs[i % copies], nbytes, part, n_wg, pattern, loads)
                        us = hip.timer_stop() * 1e3 / launches
                        rates.append(nbytes / (us * 1e-6) / 1e9)
                    hip.free(part)
                    g = float(np.median(rates))
                    key = f"{mb}MB p{pattern} u{loads} g{n_wg}"
                    out[key] = {"us": round(nbytes / (g * 1e9) * 1e6, 3), "GB/s": round(g, 1)}
                    log(f"read probe variant {key}: {out[key]['us']} us, {g:.1f} GB/s")
                    if best is None or g > out[best]["GB/s"]:
                        best = key
        out[f"{mb}MB best"] = best
        for b in bufs:
            hip.free(b)
    print(json.dumps({"read_probe_variants": out, "launch": "yule_hip_read_probe_variant, 256-thread workgroups, "
                      "back-to-back stream launches over rotating buffers, HIP events"}), flush=True)


def mfma_probe(hip, iters=4000):
    """MFMA issue rate with no memory traffic (yule_hip_mfma_probe): both f16
    shapes, 1-8 independent chains per wave, 1-2 workgroups of four waves per
    CU (one or two waves per SIMD), median of 3 timed launches after one
    warm-up.  Prints one JSON line."""
    info = hip.device_info()
    inp = hip.upload((np.random.default_rng(5).standard_normal(1024) * 0.01).astype(np.float16))
    out = {}
    for shape, flops in ((0, 16384), (1, 32768)):
        for per_cu in (1, 2):
            n_wg = info.compute_units * per_cu
            o = hip.allocate(n_wg * 1024)
            for chains in (1, 2, 4, 8):
                hip.mfma_probe(inp, o, shape, chains, n_wg, 64)
                runs = []
                for _ in range(3):
                    hip.timer_start()
                    hip.mfma_probe(inp, o, shape, chains, n_wg, iters)
                    runs.append(hip.timer_stop())
                ms = float(np.median(runs))
                tf = flops * chains * iters * 4 * n_wg / (ms * 1e-3) / 1e12
                key = f"{'16x16x32' if shape == 0 else '32x32x16'} {per_cu} wave/SIMD {chains} chains"
                # each SIMD runs per_cu waves of chains * iters MFMAs
                out[key] = {"TFLOP/s": round(tf, 1), "mfma_per_us_per_simd": round(per_cu * chains * iters / (ms * 1e3), 2)}
                log(f"mfma probe {key}: {tf:.1f} TFLOP/s")
            hip.free(o)
    hip.free(inp)
    print(json.dumps({"mfma_probe": out, "iters": iters}), flush=True)


def profile_gemm(hip, n, M=2048):
    """N launches of the Q4_K 14336x4096 prefill GEMM at M tokens (BASELINE
    M in {64, 512, 2048}), for rocprofv3 kernel-trace and MFMA
    counter runs."""
    n_rows, n_cols = 14336, 4096
    w = hip.upload(synth.gen_quant(DType.Q4_K, 81, n_rows, n_cols))
    xb = (synth.gauss(82, (M, n_cols)).view(np.uint32) >> 16).astype(np.uint16)
    hx, hy = hip.upload(xb), hip.allocate(4 * M * n_rows)
    hip.timer_start()
    for _ in range(n):
        hip.quantized_gemm(w, hx, hy, M, n_rows, n_cols, DType.Q4_K)
    ms = hip.timer_stop() / n
    print(json.dumps({"launches": n, "us_per_call": round(ms * 1e3, 1),
                      "TFLOP/s": round(2.0 * M * n_rows * n_cols / (ms * 1e-3) / 1e12, 1)}), flush=True)


def profile_decode(hip, n):
    """N greedy decode steps of the TinyLlama-shaped model after the bench's
    128-token prompt (positions 128.., as the bench decodes), with the
    runner's kernels launched one by one (tracing profilers do not follow
    graph replays)."""
    os.environ["YULE_RUNNER_NO_GRAPH"] = "1"   # read by the runner at its first step
    from yule_amd.backend import HipRunner
    from yule_amd.model import TINYLLAMA, SyntheticModel
    model = SyntheticModel.generate(TINYLLAMA, seed=0)
    run = HipRunner(hip, model)
    toks, ms = run.generate_greedy(synth.uniform_tokens(1, 128, TINYLLAMA.vocab), n)
    run.close()
    print(json.dumps({"steps": n, "ms_per_step_ungraphed": round(ms, 4)}), flush=True)


def profile_prefill(hip, n):
    """N batched prefills of the 128-token prompt through the TinyLlama-shaped
    runner (each projection one f32-input GEMM), for rocprofv3."""
    from yule_amd.backend import HipRunner
    from yule_amd.model import TINYLLAMA, SyntheticModel
    model = SyntheticModel.generate(TINYLLAMA, seed=0)
    prompt = synth.uniform_tokens(1, 128, TINYLLAMA.vocab)
    run = HipRunner(hip, model)
    hip.synchronize()
    hip.timer_start()
    for _ in range(n):
        run.reset()
        run.prefill_batched(prompt)
    ms = hip.timer_stop() / n
    run.close()
    print(json.dumps({"prefills": n, "ms_per_prefill": round(ms, 3),
                      "prefill_tok_s": round(len(prompt) * 1000.0 / ms, 1)}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--copies", type=int, default=8)
    ap.add_argument("--repeats", type=int, default=7,
                    help="timed K-step runs of the headline; the median is reported")
    ap.add_argument("--quick", action="store_true", help="primary metric and roofline only")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch kernels one by one instead of replaying a HIP graph (for profilers)")
    ap.add_argument("--profile-dominant", type=int, default=0, metavar="N",
                    help="only run N launches of the dominant kernel (Q4_K 14336x4096 over rotating copies) and "
                         "one 64 MiB device copy, for rocprofv3 --pmc runs; prints a JSON line")
    ap.add_argument("--profile-gemm", type=int, default=0, metavar="N",
                    help="only run N calls of the Q4_K 14336x4096 prefill GEMM (for rocprofv3)")
    ap.add_argument("--gemm-m", type=int, default=2048, choices=(1, 16, 32, 64, 512, 2048),
                    help="tokens M of the --profile-gemm calls (default 2048; M <= 32 runs the few-rows kernel)")
    ap.add_argument("--probe-curve", action="store_true",
                    help="only measure the single-launch streaming-read rate against launch size (JSON line)")
    ap.add_argument("--probe-variants", action="store_true",
                    help="only measure the single-launch read rate by access pattern and grid (JSON line)")
    ap.add_argument("--mfma-probe", action="store_true", help="only measure the MFMA issue rate (JSON line)")
    ap.add_argument("--profile-decode", type=int, default=0, metavar="N",
                    help="only run N TinyLlama decode steps with kernels launched one by one (for rocprofv3)")
    ap.add_argument("--profile-prefill", type=int, default=0, metavar="N",
                    help="only run N batched 128-token TinyLlama prefills (for rocprofv3)")
    args = ap.parse_args()
    global USE_GRAPH
    USE_GRAPH = not args.no_graph
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the matvec shards by "
              f"rows with no exchange, so N GPUs would each run 1/N of every projection.", file=sys.stderr)
        sys.exit(2)

    from yule_amd.backend import HipBackend
    hip = HipBackend(0)
    info = hip.device_info()
    if args.profile_dominant:
        profile_dominant(hip, args.profile_dominant, args.copies)
        return
    if args.probe_curve:
        probe_curve(hip)
        return
    if args.mfma_probe:
        mfma_probe(hip)
        return
    if args.probe_variants:
        probe_variants(hip)
        return
    if args.profile_gemm:
        profile_gemm(hip, args.profile_gemm, args.gemm_m)
        return
    if args.profile_decode:
        profile_decode(hip, args.profile_decode)
        return
    if args.profile_prefill:
        profile_prefill(hip, args.profile_prefill)
        return
    log(f"device: {info.name}, {info.compute_units} CUs, {info.memory_bytes / 2**30:.0f} GiB")

    log("generating Llama-3-8B Q4_K layer")
    q4k = Layer(hip, DType.Q4_K, LLAMA3_LAYER, args.copies, seed=11)

    # warm-up steps, then exactly K timed steps, repeated: the median timing
    # is the headline, the others its spread
    time_steps(hip, q4k, args.warmup)
    reps = sorted(time_steps(hip, q4k, args.steps) for _ in range(max(1, args.repeats)))
    ms = reps[len(reps) // 2]
    ms_per_step = ms / args.steps
    value = q4k.step_bytes * args.steps / (ms * 1e-3) / 1e9
    rep_values = [round(q4k.step_bytes * args.steps / (m * 1e-3) / 1e9, 1) for m in reps]
    log(f"Q4_K layer: {ms_per_step * 1e3:.2f} us/step, {value:.1f} GB/s ({100 * value / HBM_PEAK_GBS:.1f}% of peak); "
        f"repeats {rep_values}")
    ms7 = time_steps(hip, q4k, args.steps, fused=False)
    value7 = q4k.step_bytes * args.steps / (ms7 * 1e-3) / 1e9
    log(f"Q4_K layer as 7 separate calls: {value7:.1f} GB/s")

    # dominant kernel: Q4_K 14336x4096 (gate/up), average launch duration over
    # DOM_COPIES distinct copies (1.06 GB, four times the 256 MB last-level
    # cache, so no launch finds its weights cached)
    n_dom = 1000
    dom = Layer(hip, DType.Q4_K, [("ffn_gate", 14336, 4096)], DOM_COPIES, seed=11)
    us, gbs, dom_runs = dominant_rate(hip, dom, n_dom)
    dom_bytes = algo_bytes(DType.Q4_K, 14336, 4096)
    roofline = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(),
                "kernel": f"{dominant_kernel_name()} 14336x4096", "avg_launch_us": round(us, 3),
                "avg_launch_us_passes": [round(u, 3) for u in dom_runs],
                "algo_bytes_per_launch": dom_bytes, "profile_avg_us": profile_avg_us()}
    if roofline["profile_avg_us"]:   # the committed rocprofv3 trace of this same loop
        roofline["frac_trace"] = round(dom_bytes / (roofline["profile_avg_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
    log(f"dominant kernel Q4_K 14336x4096: {us:.2f} us/launch, {gbs:.1f} GB/s")
    roofline["read_probe"] = read_probe(hip, dom, "ffn_gate", n_dom)
    # the fastest single-launch read pattern of the variant sweep (bench.py --probe-variants)
    roofline["read_probe_best"] = read_probe(hip, dom, "ffn_gate", n_dom, n_wg=1024, pattern=1, loads=2)
    roofline["weight_copies"] = DOM_COPIES
    dom.free()
    best = max(roofline["read_probe"]["GB/s"], roofline["read_probe_best"]["GB/s"])
    roofline["frac_of_read_probe"] = round(gbs / best, 4)
    log(f"read probe over the same weight copies: {roofline['read_probe']['us']:.2f} us/launch "
        f"(best variant {roofline['read_probe_best']['us']:.2f} us), {best:.1f} GB/s")

    # fixed cost of the step's kernel boundaries: the same number of empty
    # kernels per step, replayed from one graph like the timed steps
    n_launch = len(q4k.ops_for_step(0))
    hip.time_empty_launches(n_launch * min(args.steps, 64), 1, use_graph=USE_GRAPH)        # warm-up
    empty_ms = hip.time_empty_launches(n_launch * args.steps, 1, use_graph=USE_GRAPH)   # one graph, as the steps
    launch_us = 1e3 * empty_ms / args.steps
    extra = {"headline_repeats": {"n": len(reps), "GB/s": rep_values[::-1],
                                  "spread_pct": round(100 * (rep_values[0] - rep_values[-1]) / value, 2)},
             "layer_as_7_calls_GB/s": round(value7, 1), "per_matrix_q4k": {},
             "launch_overhead": {"empty_kernels_per_step": n_launch, "us_per_step": round(launch_us, 3),
                                 "value_without_it_GB/s": round(q4k.step_bytes / ((ms_per_step * 1e3 - launch_us) * 1e-6) / 1e9, 1)}}
    log(f"empty-kernel step ({n_launch} launches): {launch_us:.2f} us")
    for name, r, c in LLAMA3_LAYER:
        u, g = matrix_rate(hip, q4k, name, 400)
        extra["per_matrix_q4k"][f"{name} {r}x{c}"] = {"us": round(u, 2), "GB/s": round(g, 1)}

    cpu = None if args.no_cpu else cpu_baseline(q4k)
    if cpu:
        log(f"CPU baseline: {cpu['value']} GB/s on {cpu['cores']} threads ({cpu['host_cpu']})")
    q4k.free()

    e2e = decode_e2e(hip, cpu=not args.no_cpu)
    log(f"TinyLlama Q4_K_M decode: {e2e['decode_tok_s']} tok/s ({e2e['decode_ms_per_step']} ms/step)"
        + (f", CPU {e2e['cpu_decode']['tok_s']} tok/s" if "cpu_decode" in e2e else ""))
    extra.update(e2e)

    if not args.quick:
        extra["prefill_gemm_q4k"] = prefill_gemm(hip)
        # a few X rows (M <= 32: the streaming few-rows kernel)
        extra["prefill_gemm_q4k_few_rows"] = prefill_gemm(hip, DType.Q4_K, ((14336, 4096), (4096, 14336)), (1, 16, 32))
        extra["prefill_gemm_other_formats"] = {
            dt.name: prefill_gemm(hip, dt, ((14336, 4096),), (512, 2048))
            for dt in (DType.Q4_0, DType.Q5_K, DType.Q6_K, DType.Q8_0, DType.Q8_K)}
        for dt in (DType.Q6_K, DType.Q8_0):
            log(f"generating Llama-3-8B {dt.name} layer")
            L = Layer(hip, dt, LLAMA3_LAYER, args.copies, seed=21 + int(dt))
            n = max(64, args.steps // 4)
            time_steps(hip, L, 32)
            m = time_steps(hip, L, n)
            g = L.step_bytes * n / (m * 1e-3) / 1e9
            extra[f"llama3_layer_{dt.name.lower()}_GB/s"] = round(g, 1)
            log(f"{dt.name} layer: {g:.1f} GB/s")
            L.free()
        for dt in (DType.Q4_K, DType.Q6_K, DType.Q8_0):
            L = Layer(hip, dt, [LLAMA3_LM_HEAD], 1, seed=31 + int(dt))
            u, g = matrix_rate(hip, L, "output", 50)
            extra[f"llama3_lm_head_{dt.name.lower()}"] = {"us": round(u, 1), "GB/s": round(g, 1)}
            log(f"lm_head 128256x4096 {dt.name}: {u:.1f} us, {g:.1f} GB/s")
            L.free()
        sweep = {}
        for name, r, c, dt in TINY_SWEEP:
            L = Layer(hip, dt, [(name, r, c)], 16, seed=41)
            u, g = matrix_rate(hip, L, name, 800)
            sweep[f"{name} {r}x{c} {dt.name}"] = {"us": round(u, 2), "GB/s": round(g, 1)}
            L.free()
        extra["tinyllama_sweep"] = sweep
        # configs[1] as the runner issues it: a TinyLlama layer's Q4_K
        # projections as its four decode launches (Q/K/V multi, O, gate/up,
        # down), back to back from one graph over 64 rotating layer copies
        # (1.4 GB), and the lm_head launches back to back
        L = Layer(hip, DType.Q4_K, TINY_LAYER, 64, seed=51)
        n = max(256, args.steps)
        time_steps(hip, L, 64)
        m = time_steps(hip, L, n)
        extra["tinyllama_layer_q4k"] = {"us_per_layer": round(1e3 * m / n, 2),
                                        "GB/s": round(L.step_bytes * n / (m * 1e-3) / 1e9, 1),
                                        "launches_per_layer": len(L.ops_for_step(0)), "layer_bytes": L.step_bytes}
        log(f"TinyLlama Q4_K layer (runner launches): {1e3 * m / n:.2f} us, "
            f"{extra['tinyllama_layer_q4k']['GB/s']} GB/s")
        L.free()

    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: W ~ N(0,0.02) seeded, GGUF Q4_K blocks; x ~ N(0,1) f32",
        "config": {"workload": "Llama-3-8B layer projections, Q4_K decode matvec, batch 1 (BASELINE configs[2])",
                   "hidden": 4096, "ffn": 14336, "kv_heads": 8, "head_dim": 128, "layer_copies": args.copies,
                   "step_bytes": q4k.step_bytes},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": roofline, "cpu_baseline": cpu, "device": info.name, **extra,
    }
    hip.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
