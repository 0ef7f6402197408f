import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: runs HIP kernels on an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def dev():
    """A visible HIP device. The library itself must load: a missing build is
    an error, never a skip."""
    from swiftllm_amd import _hip, _lib

    _lib.lib()
    if _hip.device_count() < 1:
        pytest.skip("no HIP device visible")
    return 0
