import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu_device():
    """Device 0, or skip when this host has no GPU (the CPU build container)."""
    from gguf2bin_amd import hip

    if hip.device_count() < 1:
        pytest.skip("no GPU visible")
    hip.set_device(0)
    return 0
