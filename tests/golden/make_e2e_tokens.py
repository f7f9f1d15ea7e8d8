"""Write tests/golden/e2e_tinyllama_greedy.json: the greedy token stream of
the CPU oracle (oracle/runner.c, the restatement of Yule's TransformerRunner)
on the TinyLlama-shaped synthetic Q4_K_M model of BASELINE configs[4]:
model seed 0, prompt = 128 token ids from ys_uniform_u32(seed 1), then 256
decode steps (positions 128..383).  Records the argmax after the last prompt
token and after every decode step (257 ids), each step's top-1/top-2 logit
margin, and the sha256 digest of the model bytes (so a GPU run can check
that it regenerated the same model).

    python tests/golden/make_e2e_tokens.py [--threads N]
"""
import argparse
import json
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path[:0] = [str(HERE.parent.parent), str(HERE.parent)]

import oracle  # noqa: E402
from yule_amd import synth  # noqa: E402
from yule_amd.model import TINYLLAMA, SyntheticModel  # noqa: E402

N_PROMPT, N_DECODE, MODEL_SEED, PROMPT_SEED = 128, 256, 0, 1


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=0)
    a = ap.parse_args()
    t0 = time.time()
    m = SyntheticModel.generate(TINYLLAMA, seed=MODEL_SEED)
    digest = m.digest()
    print(f"model generated in {time.time() - t0:.1f}s, digest {digest[:16]}", flush=True)
    prompt = synth.uniform_tokens(PROMPT_SEED, N_PROMPT, TINYLLAMA.vocab)
    r = oracle.Runner(m, n_threads=a.threads)
    toks, margins = [], []
    t0 = time.time()
    logits = None
    for t in prompt:
        logits = r.forward(int(t))
    for step in range(N_DECODE + 1):
        nxt = oracle.argmax(logits)
        top2 = np.sort(logits)[-2:]
        toks.append(nxt)
        margins.append(float(top2[1] - top2[0]))
        if step < N_DECODE:
            logits = r.forward(nxt)
    dt = time.time() - t0
    out = {"config": "TinyLlama-shaped (BASELINE configs[4])", "model_seed": MODEL_SEED, "prompt_seed": PROMPT_SEED,
           "n_prompt": N_PROMPT, "n_decode": N_DECODE, "model_sha256": digest,
           "prompt": [int(t) for t in prompt], "tokens": [int(t) for t in toks], "top2_margin": margins,
           "oracle_seconds": round(dt, 1)}
    (HERE / "e2e_tinyllama_greedy.json").write_text(json.dumps(out))
    print(f"{len(toks)} tokens in {dt:.1f}s; min margin {min(margins):.3g}; first {toks[:8]}")


if __name__ == "__main__":
    main()
