import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libyule_hip.so")


@pytest.fixture(scope="session")
def hip():
    """One HipBackend for the whole GPU session (raises if the HIP path is unavailable:
    there is no CPU fallback to hide behind)."""
    from yule_amd.backend import HipBackend
    be = HipBackend(0)
    yield be
    be.close()
