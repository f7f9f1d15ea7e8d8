"""Child-process check for tests/test_runner_gpu.py: the batched prefill with
the GEMM's K split forced to a given count (YULE_GEMM_SPLITS, read once per
process, set by the parent).  With one split every projection stores its
tiles straight from the epilogue, so the output and down products add into
the residual rows there instead of in the split-K reduction.  A two-layer
model's 40-token batch, then 8 decode steps, logits vs the oracle.  Prints
one line: "ok <max err / bar>" or raises."""
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path[:0] = [str(ROOT), str(ROOT / "tests")]

import numpy as np  # noqa: E402

import oracle  # noqa: E402
from refgen import tolerance_bar  # noqa: E402
from yule_amd import synth  # noqa: E402
from yule_amd.backend import HipBackend, HipRunner  # noqa: E402
from yule_amd.model import LlamaConfig, SyntheticModel  # noqa: E402

CFG = LlamaConfig(n_layers=2, dim=512, n_heads=8, n_kv_heads=2, ff_dim=1024, vocab=1024, max_seq=64)


def main():
    m = SyntheticModel.generate(CFG, seed=29)
    toks = synth.uniform_tokens(44, 48, CFG.vocab)
    worst = 0.0
    with HipBackend(0) as hip:
        run, ref = HipRunner(hip, m), oracle.Runner(m, n_threads=4)
        got = run.prefill_batched(toks[:40])
        for t in toks[:40]:
            want = ref.forward(int(t))
        worst = max(worst, float(np.max(np.abs(got - want))) / tolerance_bar(want))
        for t in toks[40:]:
            got, want = run.decode_step(int(t)), ref.forward(int(t))
            worst = max(worst, float(np.max(np.abs(got - want))) / tolerance_bar(want))
        run.close()
    if not worst <= 1.0:
        raise AssertionError(f"max err / bar {worst:.3f}")
    print(f"ok {worst:.3f}")


if __name__ == "__main__":
    main()
