import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) visible to HIP")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def hip():
    """The loaded gfx950 library with a device; fails (never skips) when a
    GPU test runs without one, so a missing backend cannot pass silently."""
    from cortexmind_amd import _lib
    from cortexmind_amd.device import device_count, device_info

    _lib.lib()
    assert device_count() >= 1, "GPU test run without a visible HIP device"
    info = device_info()
    assert "gfx950" in info["arch"], f"expected gfx950, got {info}"
    return _lib
