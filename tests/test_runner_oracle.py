"""CPU checks of the oracle's TransformerRunner restatement (oracle/runner.c)."""
import numpy as np

import oracle
from np_forward import NpForward
from yule_amd import synth
from yule_amd.model import TINY_TEST, SyntheticModel


def _model():
    return SyntheticModel.generate(TINY_TEST, seed=3)


def test_oracle_runner_matches_f64_forward():
    m = _model()
    r, ref = oracle.Runner(m, n_threads=2), NpForward(m)
    toks = synth.uniform_tokens(5, 12, m.cfg.vocab)
    for t in toks:
        got, want = r.forward(int(t)), ref.forward(int(t))
        assert np.max(np.abs(got - want)) <= 1e-3 * np.linalg.norm(want) / np.sqrt(want.size)


def test_oracle_runner_prefill_determinism_and_reset():
    """yule-validate correctness.rs:1026-1092 (prefill determinism) and :1097-1204 (reset)."""
    m = _model()
    r = oracle.Runner(m, n_threads=2)
    toks = synth.uniform_tokens(6, 20, m.cfg.vocab)
    a = [r.forward(int(t)) for t in toks]
    r.reset()
    assert r.pos == 0
    b = [r.forward(int(t)) for t in toks]
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_oracle_runner_context_limit():
    m = _model()
    r = oracle.Runner(m, n_threads=1)
    for i in range(m.cfg.max_seq):
        r.forward(i % m.cfg.vocab)
    try:
        r.forward(0)
    except RuntimeError:
        return
    raise AssertionError("forward past max_seq must fail (model_runner.rs:538-540)")
