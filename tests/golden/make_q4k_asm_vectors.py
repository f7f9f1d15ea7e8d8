"""Write tests/golden/q4k_asm_vectors.npz: the reference's own Q4_K AVX2
assembly kernel (yule-core/src/kernels/q4k_gemv_avx2.S, assembled from the
reference tree into oracle/_ref/ by `make -C oracle ref`) evaluated on the
first 64 block/activation pairs of the reference's Q4_K differential-test
generator (yule-core/src/simd/avx2.rs:419-441, xorshift seed 777).

Run in a container that has the reference tree:  python tests/golden/make_q4k_asm_vectors.py
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path[:0] = [str(HERE.parent.parent), str(HERE.parent)]

import oracle  # noqa: E402
from refgen import xorshift_blocks  # noqa: E402

asm = oracle.q4k_asm()
if asm is None:
    sys.exit("oracle/_ref/libyule_q4k_asm.so not built (make -C oracle ref)")
blocks, acts = zip(*xorshift_blocks("q4_k", 64))
blocks, acts = np.stack(blocks), np.stack(acts)
dots = np.array([asm(blocks[i].ctypes.data, acts[i].ctypes.data) for i in range(len(blocks))], np.float32)
np.savez_compressed(HERE / "q4k_asm_vectors.npz", blocks=blocks, acts=acts, asm_dot=dots)
print("wrote", len(dots), "vectors; first", dots[:4])
