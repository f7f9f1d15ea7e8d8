"""GPU decode runner (yule_hip_runner_*) against the CPU oracle's
TransformerRunner restatement: per-step logits within the matvec bar, and
greedy tokens identical — on a small model live, and on the TinyLlama-shaped
Q4_K_M model against the committed golden stream."""
import json
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle
from np_forward import NpForward
from refgen import GOLDEN, tolerance_bar
from yule_amd import synth
from yule_amd.backend import HipRunner, YuleGpuError
from yule_amd.model import TINY_TEST, TINYLLAMA, SyntheticModel

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def tiny():
    return SyntheticModel.generate(TINY_TEST, seed=3)


@pytest.mark.parametrize("fused,split_min", [(True, None), (False, None), (True, "1"), (True, "20")],
                         ids=["fused", "unfused", "split", "split-from-20"])
def test_runner_logits_match_oracle_small(hip, tiny, fused, split_min, monkeypatch):
    """Both step sequences: fused (norm/SwiGLU staged into the matvec, residual
    and argmax epilogues) and the plain kernel-per-operation sequence; and
    attention split-KV on every step, or from position 19 on (the runner
    switching graphs mid-sequence)."""
    say(f"[runner] small model logits vs oracle ({'fused' if fused else 'unfused'}, split from {split_min})")
    if not fused:
        monkeypatch.setenv("YULE_RUNNER_UNFUSED", "1")
    if split_min:
        monkeypatch.setenv("YULE_ATTN_SPLIT_MIN", split_min)
    run = HipRunner(hip, tiny)
    ref, f64 = oracle.Runner(tiny, n_threads=4), NpForward(tiny)
    for t in synth.uniform_tokens(11, 40, tiny.cfg.vocab):
        got, want, exact = run.decode_step(int(t)), ref.forward(int(t)), f64.forward(int(t))
        assert np.max(np.abs(got - want)) <= tolerance_bar(want)
        assert np.max(np.abs(got - exact)) <= tolerance_bar(exact)
    run.close()


@pytest.mark.parametrize("scheme", ["Q4_0", "Q8_0", "Q6_K", "Q5_K", "Q8_K"])
def test_runner_uniform_formats_match_oracle(hip, scheme):
    """Models whose every matrix (embedding, projections, lm_head) is one
    format: per-step logits within the bar, then greedy tokens identical.
    Q8_K has no vec_dot in the reference (scalar.rs:4-22), so Yule's CPU
    runner cannot run it; its reference is the f64 forward over the
    bit-exact dequantized weights."""
    say(f"[runner] small {scheme} model vs oracle")
    m = SyntheticModel.generate(TINY_TEST, seed=7, scheme=scheme)

    def reference():
        return NpForward(m) if scheme == "Q8_K" else oracle.Runner(m, n_threads=4)
    run = HipRunner(hip, m)
    try:
        ref = reference()
        for t in synth.uniform_tokens(13, 12, m.cfg.vocab):
            got, want = run.decode_step(int(t)), ref.forward(int(t))
            assert np.max(np.abs(got - want)) <= tolerance_bar(want)
    finally:
        run.close()
    prompt = synth.uniform_tokens(14, 8, m.cfg.vocab)
    n_dec = 24
    run = HipRunner(hip, m)
    try:
        toks, _ = run.generate_greedy(prompt, n_dec)
    finally:
        run.close()
    ref = reference()
    for t in prompt:
        logits = ref.forward(int(t))
    want = []
    for i in range(n_dec + 1):
        want.append(oracle.argmax(logits))
        if i < n_dec:
            logits = ref.forward(want[-1])
    assert list(toks) == want


def test_runner_greedy_matches_oracle_small(hip, tiny):
    say("[runner] small model greedy tokens vs oracle")
    prompt = synth.uniform_tokens(12, 20, tiny.cfg.vocab)
    n_dec = tiny.cfg.max_seq - prompt.size
    run = HipRunner(hip, tiny)
    toks, ms = run.generate_greedy(prompt, n_dec)
    ref = oracle.Runner(tiny, n_threads=4)
    for t in prompt:
        logits = ref.forward(int(t))
    want = []
    for i in range(n_dec + 1):
        want.append(oracle.argmax(logits))
        if i < n_dec:
            logits = ref.forward(want[-1])
    assert list(toks) == want
    assert ms > 0
    run.close()


HD64 = None


@pytest.mark.parametrize("chunks,split_min", [("1", None), ("1", "100"), ("0", None)],
                         ids=["chunked", "chunked-then-split", "per-head"])
def test_runner_hd64_attention_paths(hip, chunks, split_min, monkeypatch):
    """Head size 64 on narrow teams: the Q/K/V launch applies RoPE and writes
    the cache (kEpiRope) and attention runs chunked with its in-launch
    combine, over 1..150 positions (one to three 64-position chunks); then the
    same with split-KV from position 99 on, and with the one-workgroup-per-head
    kernel.  Logits vs the oracle and the float64 forward at every step, then
    greedy tokens."""
    from yule_amd.model import LlamaConfig
    global HD64
    if HD64 is None:
        HD64 = SyntheticModel.generate(LlamaConfig(n_layers=2, dim=512, n_heads=8, n_kv_heads=2, ff_dim=1024,
                                                   vocab=1024, max_seq=160), seed=9)
    m = HD64
    say(f"[runner] hd 64 model, chunked attention {chunks}, split from {split_min}")
    monkeypatch.setenv("YULE_ATTN_CHUNKS", chunks)
    if split_min:
        monkeypatch.setenv("YULE_ATTN_SPLIT_MIN", split_min)
    run = HipRunner(hip, m)
    ref, f64 = oracle.Runner(m, n_threads=4), NpForward(m)
    toks = synth.uniform_tokens(31, 150, m.cfg.vocab)
    for i, t in enumerate(toks):
        got, want, exact = run.decode_step(int(t)), ref.forward(int(t)), f64.forward(int(t))
        assert np.max(np.abs(got - want)) <= tolerance_bar(want), f"step {i}"
        assert np.max(np.abs(got - exact)) <= tolerance_bar(exact), f"step {i}"
    run.close()
    prompt = synth.uniform_tokens(32, 70, m.cfg.vocab)
    run = HipRunner(hip, m)
    out, _ = run.generate_greedy(prompt, 80)
    run.close()
    ref = oracle.Runner(m, n_threads=4)
    for t in prompt:
        logits = ref.forward(int(t))
    want = []
    for i in range(81):
        want.append(oracle.argmax(logits))
        if i < 80:
            logits = ref.forward(want[-1])
    assert [int(t) for t in out] == want


@pytest.mark.parametrize("scheme,dim,hd", [("Q4_K", 512, 64), ("Q6_K", 1024, 64), ("Q8_0", 512, 128),
                                            ("Q6_K", 512, 128), ("Q4_K", 2048, 128)])
def test_runner_attention_formats_and_head_sizes(hip, scheme, dim, hd):
    """The decode step with RoPE and the cache write in the Q/K/V launch and
    chunked attention, on Q4_K, Q6_K and Q8_0 Q/K/V, head sizes 64 and 128
    and both narrow team widths (16 and 32 lanes), over 1..140 positions:
    logits vs the oracle at every step, then greedy tokens vs the oracle."""
    from yule_amd.model import LlamaConfig
    cfg = LlamaConfig(n_layers=1, dim=dim, n_heads=dim // hd, n_kv_heads=2, ff_dim=512, vocab=512, max_seq=200)
    m = SyntheticModel.generate(cfg, seed=21, scheme=scheme)
    say(f"[runner] attention paths, {scheme} dim {dim} hd {hd}")
    toks = synth.uniform_tokens(33, 140, cfg.vocab)
    run = HipRunner(hip, m)
    ref = oracle.Runner(m, n_threads=4)
    try:
        for i, t in enumerate(toks):
            got, want = run.decode_step(int(t)), ref.forward(int(t))
            assert np.max(np.abs(got - want)) <= tolerance_bar(want), f"step {i}"
    finally:
        run.close()
    prompt = synth.uniform_tokens(34, 20, cfg.vocab)
    run = HipRunner(hip, m)
    out, _ = run.generate_greedy(prompt, 60)
    run.close()
    ref = oracle.Runner(m, n_threads=4)
    for t in prompt:
        logits = ref.forward(int(t))
    want = []
    for i in range(61):
        want.append(oracle.argmax(logits))
        if i < 60:
            logits = ref.forward(want[-1])
    assert [int(t) for t in out] == want


@pytest.mark.parametrize("mask,wgs", [("7", "64"), ("7", "256"), ("0", "256")])
def test_runner_prefetch_workgroups(hip, monkeypatch, mask, wgs):
    """Decode with prefetch workgroups on every pairing the runner offers (O
    -> gate/up, gate/up -> down, Q/K/V -> O), none, and a small prefetch
    grid: logits of 6 steps vs the oracle, then greedy tokens vs the
    oracle.  TinyLlama widths (2048 / 5632) so that every consumer grid maps
    row groups to XCDs and the prefetch is planned."""
    from yule_amd.model import LlamaConfig
    monkeypatch.setenv("YULE_RUNNER_PREFETCH", mask)
    monkeypatch.setenv("YULE_RUNNER_PREFETCH_WGS", wgs)
    cfg = LlamaConfig(n_layers=2, dim=2048, n_heads=32, n_kv_heads=4, ff_dim=5632, vocab=512, max_seq=64)
    m = SyntheticModel.generate(cfg, seed=27, scheme="Q4_K")
    say(f"[runner] prefetch mask {mask}, {wgs} workgroups")
    run = HipRunner(hip, m)
    ref = oracle.Runner(m, n_threads=4)
    try:
        for i, t in enumerate(synth.uniform_tokens(37, 6, cfg.vocab)):
            got, want = run.decode_step(int(t)), ref.forward(int(t))
            assert np.max(np.abs(got - want)) <= tolerance_bar(want), f"step {i}"
    finally:
        run.close()
    prompt = synth.uniform_tokens(38, 5, cfg.vocab)
    run = HipRunner(hip, m)
    out, _ = run.generate_greedy(prompt, 20)
    run.close()
    ref = oracle.Runner(m, n_threads=4)
    for t in prompt:
        logits = ref.forward(int(t))
    want = []
    for i in range(21):
        want.append(oracle.argmax(logits))
        if i < 20:
            logits = ref.forward(want[-1])
    assert [int(t) for t in out] == want


def test_runner_three_wave_team_rows(hip):
    """Rows of 176 units (Q8_0, 5632 columns) run on three-wave teams in
    every matvec of the step: RMSNorm staging into Q/K/V, gate and up
    (unpaired: paired rows need one-wave teams) and the lm_head argmax, the
    SwiGLU staging into down, the residual add on O and down.  Logits of 10
    steps vs the oracle, then greedy tokens vs the oracle."""
    from yule_amd.model import LlamaConfig
    cfg = LlamaConfig(n_layers=1, dim=5632, n_heads=44, n_kv_heads=4, ff_dim=5632, vocab=512, max_seq=64)
    m = SyntheticModel.generate(cfg, seed=23, scheme="Q8_0")
    say("[runner] three-wave teams, Q8_0 dim 5632")
    run = HipRunner(hip, m)
    ref = oracle.Runner(m, n_threads=4)
    try:
        for i, t in enumerate(synth.uniform_tokens(35, 10, cfg.vocab)):
            got, want = run.decode_step(int(t)), ref.forward(int(t))
            assert np.max(np.abs(got - want)) <= tolerance_bar(want), f"step {i}"
    finally:
        run.close()
    prompt = synth.uniform_tokens(36, 6, cfg.vocab)
    run = HipRunner(hip, m)
    out, _ = run.generate_greedy(prompt, 12)
    run.close()
    ref = oracle.Runner(m, n_threads=4)
    for t in prompt:
        logits = ref.forward(int(t))
    want = []
    for i in range(13):
        want.append(oracle.argmax(logits))
        if i < 12:
            logits = ref.forward(want[-1])
    assert [int(t) for t in out] == want


@pytest.mark.parametrize("which", ["tiny", "hd64"])
def test_runner_prefill_batched_matches_oracle(hip, tiny, which):
    """The prompt as one batched pass (GEMM projections, causal attention
    per row): last-token logits vs the oracle's token-by-token prefill, a
    second batch from position 20 on, then decode steps over the cache the
    batches wrote."""
    from yule_amd.model import LlamaConfig
    global HD64
    if which == "hd64" and HD64 is None:
        HD64 = SyntheticModel.generate(LlamaConfig(n_layers=2, dim=512, n_heads=8, n_kv_heads=2, ff_dim=1024,
                                                   vocab=1024, max_seq=160), seed=9)
    m = tiny if which == "tiny" else HD64
    say(f"[runner] batched prefill vs oracle ({which})")
    toks = synth.uniform_tokens(41, 44, m.cfg.vocab)
    run, ref = HipRunner(hip, m), oracle.Runner(m, n_threads=4)
    got = run.prefill_batched(toks[:20])
    for t in toks[:20]:
        want = ref.forward(int(t))
    assert run.pos == 20
    assert np.max(np.abs(got - want)) <= tolerance_bar(want)
    got = run.prefill_batched(toks[20:37])
    for t in toks[20:37]:
        want = ref.forward(int(t))
    assert np.max(np.abs(got - want)) <= tolerance_bar(want)
    for i, t in enumerate(toks[37:]):
        got, want = run.decode_step(int(t)), ref.forward(int(t))
        assert np.max(np.abs(got - want)) <= tolerance_bar(want), f"decode step {i}"
    run.close()


@pytest.mark.parametrize("scheme,dim,hd", [("Q6_K", 512, 64), ("Q8_0", 512, 128), ("Q4_0", 256, 32),
                                            ("Q5_K", 512, 64), ("Q8_K", 512, 128)])
def test_runner_prefill_batched_formats(hip, scheme, dim, hd):
    """Batched prefill on every GEMM format and head sizes 32 to 128: a
    one-token batch, a 33-token batch (ragged against the GEMM's 64-row
    tiles), then decode steps over the cache they wrote; logits vs the
    oracle (Q8_K, which Yule's CPU runner cannot run: the float64 forward).
    An empty batch and one past the context length are refused."""
    from yule_amd.model import LlamaConfig
    cfg = LlamaConfig(n_layers=2, dim=dim, n_heads=dim // hd, n_kv_heads=2, ff_dim=512, vocab=512, max_seq=96)
    m = SyntheticModel.generate(cfg, seed=23, scheme=scheme)
    say(f"[runner] batched prefill, {scheme} dim {dim} hd {hd}")
    ref = NpForward(m) if scheme == "Q8_K" else oracle.Runner(m, n_threads=4)
    toks = synth.uniform_tokens(42, 44, cfg.vocab)
    run = HipRunner(hip, m)
    try:
        got, want = run.prefill_batched(toks[:1]), ref.forward(int(toks[0]))
        assert np.max(np.abs(got - want)) <= tolerance_bar(want)
        got = run.prefill_batched(toks[1:34])
        for t in toks[1:34]:
            want = ref.forward(int(t))
        assert run.pos == 34
        assert np.max(np.abs(got - want)) <= tolerance_bar(want)
        for i, t in enumerate(toks[34:]):
            got, want = run.decode_step(int(t)), ref.forward(int(t))
            assert np.max(np.abs(got - want)) <= tolerance_bar(want), f"decode step {i}"
        with pytest.raises(YuleGpuError):
            run.prefill_batched(np.zeros(0, np.uint32))
        with pytest.raises(YuleGpuError, match="context"):
            run.prefill_batched(synth.uniform_tokens(43, cfg.max_seq - run.pos + 1, cfg.vocab))
        assert run.pos == 44
    finally:
        run.close()


def test_runner_greedy_token_prefill_path(hip, tiny, monkeypatch):
    """generate_greedy with the token-by-token prompt pass (the runner's
    fallback when a projection has no batched path) gives the oracle's tokens,
    as the batched pass does."""
    say("[runner] greedy with token-by-token prefill")
    prompt = synth.uniform_tokens(43, 24, tiny.cfg.vocab)
    outs = []
    for env in ("1", None):
        if env:
            monkeypatch.setenv("YULE_RUNNER_TOKEN_PREFILL", env)
        else:
            monkeypatch.delenv("YULE_RUNNER_TOKEN_PREFILL", raising=False)
        run = HipRunner(hip, tiny)
        outs.append([int(t) for t in run.generate_greedy(prompt, 30)[0]])
        run.close()
    ref = oracle.Runner(tiny, n_threads=4)
    for t in prompt:
        logits = ref.forward(int(t))
    want = []
    for i in range(31):
        want.append(oracle.argmax(logits))
        if i < 30:
            logits = ref.forward(want[-1])
    assert outs[0] == want and outs[1] == want


@pytest.mark.parametrize("threads_w64", ["256", "512"])
def test_runner_wide_rows_fused_variants(hip, threads_w64):
    """4096-wide rows: every fused matvec variant on one-wave teams, in both
    workgroup sizes the launcher can pick for them (tests/runner_wide_check.py,
    in a child process because the size is read once per process)."""
    import os
    import subprocess
    say(f"[runner] 4096-wide model, one-wave teams in {threads_w64}-thread workgroups")
    env = dict(os.environ, YULE_QMV_THREADS_W64=threads_w64)
    r = subprocess.run([sys.executable, str(Path(__file__).with_name("runner_wide_check.py"))], env=env,
                       capture_output=True, text=True, timeout=110)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout[-2000:] + r.stderr[-4000:]
    say(f"[runner] {r.stdout.strip()}")


@pytest.mark.parametrize("splits", ["1", "3"])
def test_runner_prefill_batched_forced_splits(hip, splits):
    """The batched prefill with the GEMM's K split forced to 1 (every tile
    stored by the epilogue, which adds the O and down products into the
    residual rows) and to 3 (the split-K reduction does it), against the
    oracle (tests/prefill_splits_check.py, in a child process because the
    split count is read once per process)."""
    import os
    import subprocess
    say(f"[runner] batched prefill with {splits} K splits")
    env = dict(os.environ, YULE_GEMM_SPLITS=splits)
    r = subprocess.run([sys.executable, str(Path(__file__).with_name("prefill_splits_check.py"))], env=env,
                       capture_output=True, text=True, timeout=110)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout[-2000:] + r.stderr[-4000:]
    say(f"[runner] {r.stdout.strip()}")


def test_runner_prefill_determinism_reset_and_limits(hip, tiny):
    say("[runner] prefill determinism / reset / context limit")
    run = HipRunner(hip, tiny)
    toks = synth.uniform_tokens(13, 16, tiny.cfg.vocab)
    a = run.prefill(toks)
    assert run.pos == 16
    run.reset()
    assert run.pos == 0
    b = run.prefill(toks)
    assert np.array_equal(a, b)
    with pytest.raises(YuleGpuError):
        run.decode_step(tiny.cfg.vocab)            # token out of range
    run.reset()
    for i in range(tiny.cfg.max_seq):
        run.decode_step(i % tiny.cfg.vocab)
    with pytest.raises(YuleGpuError):
        run.decode_step(0)                         # context length exceeded
    run.close()


@pytest.fixture(scope="module")
def tinyllama():
    return SyntheticModel.generate(TINYLLAMA, seed=0)


def test_tinyllama_first_steps_logits_vs_oracle(hip, tinyllama):
    say("[runner] TinyLlama first decode steps vs oracle logits")
    g = json.loads((GOLDEN / "e2e_tinyllama_greedy.json").read_text())
    run = HipRunner(hip, tinyllama)
    ref = oracle.Runner(tinyllama)
    for t in g["prompt"][:4]:
        got, want = run.decode_step(t), ref.forward(t)
        assert np.max(np.abs(got - want)) <= tolerance_bar(want)
    run.close()


def test_tinyllama_greedy_tokens_match_golden(hip, tinyllama):
    """128-token prompt + 256 greedy decode steps; every argmax identical to the
    oracle's stream (tests/golden/e2e_tinyllama_greedy.json)."""
    g = json.loads((GOLDEN / "e2e_tinyllama_greedy.json").read_text())
    say("[runner] TinyLlama greedy 128+256 vs golden")
    assert tinyllama.digest() == g["model_sha256"], "synthetic model differs from the golden run's"
    run = HipRunner(hip, tinyllama)
    toks, ms = run.generate_greedy(np.array(g["prompt"], np.uint32), g["n_decode"])
    toks = [int(t) for t in toks]
    if toks != g["tokens"]:
        i = next(k for k, (a, b) in enumerate(zip(toks, g["tokens"])) if a != b)
        pytest.fail(f"first divergence at decode output {i}: gpu {toks[i]} vs oracle {g['tokens'][i]} "
                    f"(oracle top-2 margin there {g['top2_margin'][i]:.3g})")
    say(f"[runner] TinyLlama decode {ms:.3f} ms/step = {1000 / ms:.0f} tok/s")
    run.close()


def test_runner_from_gguf_matches_in_memory(hip, tiny, tmp_path):
    """yule_hip_runner_create_from_gguf over the model written as GGUF gives
    bit-identical logits and tokens to the runner built from host arrays."""
    say("[runner] small model from GGUF vs in-memory")
    p = tmp_path / "tiny.gguf"
    tiny.to_gguf(p)
    a, b = HipRunner(hip, tiny), HipRunner.from_gguf(hip, p, max_seq=tiny.cfg.max_seq)
    assert b.vocab == tiny.cfg.vocab
    for t in synth.uniform_tokens(14, 12, tiny.cfg.vocab):
        assert np.array_equal(a.decode_step(int(t)), b.decode_step(int(t)))
    a.reset(), b.reset()
    prompt = synth.uniform_tokens(15, 10, tiny.cfg.vocab)
    assert np.array_equal(a.generate_greedy(prompt, 20)[0], b.generate_greedy(prompt, 20)[0])
    a.close(), b.close()


def test_runner_from_gguf_tied_output_and_errors(hip, tiny, tmp_path):
    """No output.weight: the logits come from token_embd.weight
    (weight_loader.rs:166-170); an unsupported architecture and a missing
    tensor are refused before anything is uploaded."""
    say("[runner] GGUF tied embeddings / errors")
    from yule_amd.gguf import TensorEntry, model_metadata, write_gguf
    from yule_amd.model import SyntheticModel as SM, Tensor
    tied = dict(tiny.tensors)
    e = tied["token_embd.weight"]
    tied["output.weight"] = Tensor("output.weight", e.dtype, e.shape, e.data)
    ref = HipRunner(hip, SM(tiny.cfg, tied, tiny.scheme, tiny.seed))
    ents = [TensorEntry(t.name, int(t.dtype), t.shape, t.data) for n, t in tiny.tensors.items() if n != "output.weight"]
    p = tmp_path / "tied.gguf"
    write_gguf(p, model_metadata(tiny.cfg), ents)
    run = HipRunner.from_gguf(hip, p)          # max_seq from llama.context_length
    for t in (1, 2, 3):
        assert np.array_equal(ref.decode_step(t), run.decode_step(t))
    ref.close(), run.close()
    q = tmp_path / "arch.gguf"
    write_gguf(q, model_metadata(tiny.cfg, arch="mamba"), ents)
    with pytest.raises(YuleGpuError, match="architecture"):
        HipRunner.from_gguf(hip, q)
    r = tmp_path / "missing.gguf"
    write_gguf(r, model_metadata(tiny.cfg), [x for x in ents if x.name != "blk.1.ffn_up.weight"])
    with pytest.raises(YuleGpuError, match="blk.1.ffn_up.weight"):
        HipRunner.from_gguf(hip, r)


def test_tinyllama_from_gguf_greedy_matches_golden(hip, tinyllama, tmp_path):
    """The TinyLlama-shaped Q4_K_M model through a GGUF file: the full
    128 + 256 greedy stream equals the golden one."""
    g = json.loads((GOLDEN / "e2e_tinyllama_greedy.json").read_text())
    say("[runner] TinyLlama from GGUF greedy vs golden")
    p = tmp_path / "tinyllama.gguf"
    tinyllama.to_gguf(p)
    run = HipRunner.from_gguf(hip, p, max_seq=tinyllama.cfg.max_seq)
    toks, _ = run.generate_greedy(np.array(g["prompt"], np.uint32), g["n_decode"])
    assert [int(t) for t in toks] == g["tokens"]
    run.close()
    p.unlink()


def test_runner_long_context_split(hip):
    """A 2,600-position context (split-KV attention from position 511 on):
    greedy tokens identical to the oracle's over a 2,500-token prompt and 100
    decode steps."""
    from dataclasses import replace
    say("[runner] long context (2600) greedy vs oracle")
    m = SyntheticModel.generate(replace(TINY_TEST, max_seq=2600), seed=4)
    prompt = synth.uniform_tokens(16, 2500, m.cfg.vocab)
    run = HipRunner(hip, m)
    toks, _ = run.generate_greedy(prompt, 100)
    ref = oracle.Runner(m, n_threads=1)
    for t in prompt:
        logits = ref.forward(int(t))
    want = []
    for i in range(101):
        want.append(oracle.argmax(logits))
        if i < 100:
            logits = ref.forward(want[-1])
    assert list(toks) == want
    run.close()
