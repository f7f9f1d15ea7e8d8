"""Child-process check for tests/test_runner_gpu.py: a one-layer model with
4096-wide rows, every matrix Q4_K, so every fused matvec variant runs with
one-wave teams (RMSNorm staging into Q/K/V, residual add on O and down,
paired gate/up with SwiGLU, the lm_head argmax epilogue).  Logits of 12
steps are compared with the oracle and the float64 forward, fused and
unfused step sequences, then 16 greedy tokens with the oracle's.  Run in its
own process so that the matvec workgroup-size switch (read once per process,
YULE_QMV_THREADS_W64) takes the value the parent sets.  Prints one line:
"ok <max err / bar>" or raises."""
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path[:0] = [str(ROOT), str(ROOT / "tests")]

import numpy as np  # noqa: E402

import oracle  # noqa: E402
from np_forward import NpForward  # noqa: E402
from refgen import tolerance_bar  # noqa: E402
from yule_amd import synth  # noqa: E402
from yule_amd.backend import HipBackend, HipRunner  # noqa: E402
from yule_amd.model import LlamaConfig, SyntheticModel  # noqa: E402

WIDE = LlamaConfig(n_layers=1, dim=4096, n_heads=32, n_kv_heads=8, ff_dim=4096, vocab=2048, max_seq=32)


def main():
    m = SyntheticModel.generate(WIDE, seed=5, scheme="Q4_K")
    worst = 0.0
    with HipBackend(0) as hip:
        for fused in (True, False):
            import os
            if not fused:
                os.environ["YULE_RUNNER_UNFUSED"] = "1"
            run = HipRunner(hip, m)
            ref, f64 = oracle.Runner(m, n_threads=4), NpForward(m)
            for t in synth.uniform_tokens(21, 12, WIDE.vocab):
                got, want, exact = run.decode_step(int(t)), ref.forward(int(t)), f64.forward(int(t))
                for r in (want, exact):
                    e = float(np.max(np.abs(got - r))) / tolerance_bar(r)
                    worst = max(worst, e)
                    assert e <= 1.0, f"fused={fused}: logits off by {e:.3g} of the bar"
            run.close()
            os.environ.pop("YULE_RUNNER_UNFUSED", None)
        prompt = synth.uniform_tokens(22, 6, WIDE.vocab)
        run = HipRunner(hip, m)
        toks, _ = run.generate_greedy(prompt, 16)
        run.close()
    ref = oracle.Runner(m, n_threads=4)
    for t in prompt:
        logits = ref.forward(int(t))
    want = []
    for i in range(17):
        want.append(oracle.argmax(logits))
        if i < 16:
            logits = ref.forward(want[-1])
    assert [int(t) for t in toks] == want, (list(toks), want)
    print(f"ok {worst:.4f}", flush=True)


if __name__ == "__main__":
    main()
