import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("uefi-gpu_amd", "oracle"):
    path = os.path.join(ROOT, sub)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU through libuq.so")


@pytest.fixture(scope="session")
def gpu():
    """Initialise libuq on device 0 once per session (fails loudly without a GPU)."""
    import uq
    uq.init(0)
    yield uq
