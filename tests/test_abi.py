"""The C ABI boundary, checked on CPU: the library loads, exports every
symbol include/*.h declares, and fails loudly (no CPU fallback) without a
gfx950 device."""
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "yule_amd" / "libyule_hip.so"


def declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(yule_hip_\w+)\s*\(", text))
    return names


def test_header_declares_trait_surface():
    names = declared_symbols()
    # one entry point per ComputeBackend method (yule-gpu/src/lib.rs:21-132)
    for m in ("name", "device_info", "allocate", "free", "matmul", "softmax", "rms_norm", "rope", "silu",
              "element_mul", "add", "copy_to_device", "copy_from_device", "copy_buffer", "copy_buffer_offset",
              "synchronize", "attn_score", "attn_value", "quantized_matmul"):
        assert f"yule_hip_{m}" in names


def test_library_exports_every_declared_symbol():
    assert LIB.exists(), "libyule_hip.so not built"
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\b(yule_hip_\w+)\b", out))
    missing = declared_symbols() - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"


def test_python_mirror_binds_every_symbol():
    from yule_amd import backend
    assert set(backend._SIGS) == declared_symbols()
    backend.load_library()


def test_no_device_fails_loudly():
    """Without a gfx950 GPU the backend refuses to construct (no silent fallback)."""
    from yule_amd.backend import HipBackend, YuleGpuError, is_available
    if is_available():
        pytest.skip("a gfx950 device is present")
    with pytest.raises(YuleGpuError) as e:
        HipBackend(0)
    assert e.value.code == 3  # YULE_ERR_NO_DEVICE
