"""Build the native parts of yule_amd in-tree.

  libyule_hip.so    HIP backend (gfx950 code objects + C++ host runtime), the product
  libyule_synth.so  seeded synthetic weights / activations and GGUF quantizers
  oracle/build/liboracle.so and oracle/_ref/ (test infrastructure, via oracle/Makefile)

Every call recompiles (the driver's "does it build" check); objects go to
yule_amd/_build/.  Usage: python -m yule_amd.build [--no-oracle]
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB_HIP = PKG / "libyule_hip.so"
LIB_SYNTH = PKG / "libyule_synth.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_SOURCES = ["runtime.cpp", "qmv.hip", "ops.hip", "gemm.hip", "prefill.hip", "runner.cpp", "gguf.cpp"]

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    # packed FP32 VALU ops are kept out of every kernel of this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {' '.join(cmd)}")


def _compile_hip(src: Path) -> Path:
    out = OBJ / (src.name + ".o")
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    _run([HIPCC, *HIP_FLAGS, *lang, "-c", str(src), "-o", str(out)])
    return out


def build_hip() -> Path:
    OBJ.mkdir(exist_ok=True)
    srcs = [CSRC / s for s in HIP_SOURCES if (CSRC / s).exists()]
    keep = {s.name + ".o" for s in srcs}
    for stale in OBJ.glob("*.o"):   # objects of sources that no longer exist
        if stale.name not in keep:
            stale.unlink()
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(_compile_hip, srcs))
    tmp = LIB_HIP.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB_HIP)
    return LIB_HIP


def build_synth() -> Path:
    tmp = LIB_SYNTH.with_suffix(".so.tmp")
    _run(["gcc", "-O2", "-fPIC", "-shared", "-fopenmp", "-o", str(tmp), str(CSRC / "synth.c"), "-lm"])
    os.replace(tmp, LIB_SYNTH)
    return LIB_SYNTH


def build_oracle() -> None:
    _run(["make", "-s", "-C", str(ROOT / "oracle"), "-B", "all"])
    if Path("/root/reference/yule-core/src/kernels/q4k_gemv_avx2.S").exists():
        _run(["make", "-s", "-C", str(ROOT / "oracle"), "-B", "ref"])


def build_all(oracle: bool = True) -> None:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    build_synth()
    if oracle:
        build_oracle()
    build_hip()


if __name__ == "__main__":
    build_all(oracle="--no-oracle" not in sys.argv)
    print(f"built {LIB_HIP.name}, {LIB_SYNTH.name}" + ("" if "--no-oracle" in sys.argv else ", oracle"))
