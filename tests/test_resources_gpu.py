"""Device memory is returned: backends, their workspace, buffers and runners
created and destroyed repeatedly leave the free device memory where it was
(hipMemGetInfo, read through the HIP runtime the library itself links)."""
import ctypes as C
import sys

import numpy as np
import pytest

from yule_amd import DType, synth
from yule_amd.backend import HipBackend, HipRunner
from yule_amd.model import TINY_TEST, SyntheticModel

pytestmark = pytest.mark.gpu


def free_bytes() -> int:
    hip = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(), C.c_size_t()
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def cycle(model):
    be = HipBackend(0)
    w = be.upload(synth.gen_quant(DType.Q4_K, 5, 512, 1024))
    xb = (synth.gauss(6, (300, 1024)).view(np.uint32) >> 16).astype(np.uint16)
    hx, hy = be.upload(xb), be.allocate(4 * 300 * 512)
    be.quantized_gemm(w, hx, hy, 300, 512, 1024, DType.Q4_K)        # grows the backend workspace
    be.gqa_decode_attn(be.allocate(4 * 8 * 64), be.upload(np.zeros((600, 2 * 64), np.float32)),
                       be.upload(np.zeros((600, 2 * 64), np.float32)), be.allocate(4 * 8 * 64), 8, 2, 64, 600)
    run = HipRunner(be, model)
    run.generate_greedy(synth.uniform_tokens(3, 4, model.cfg.vocab), 4)
    run.close()
    be.synchronize()
    be.close()                                                      # frees buffers and workspace


def test_no_device_memory_growth():
    print("[resources] backend / runner create-destroy cycles", flush=True)
    sys.stdout.flush()
    model = SyntheticModel.generate(TINY_TEST, seed=2)
    cycle(model)                     # first cycle: runtime and code-object setup
    base = free_bytes()
    for _ in range(5):
        cycle(model)
    drift = base - free_bytes()
    assert drift < 16 << 20, f"free device memory fell by {drift} bytes over 5 cycles"
