"""The C++ host layer (include/cortex_hip.hpp) end to end on the GPU: runs
tests/cpp/host_api_test, built by __graft_entry__.build() with g++ against
the in-tree library, which checks reduce / Broadcast / matrix_t /
activation results against values it computes itself (exact integers)."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "host_api_test")

pytestmark = pytest.mark.gpu


def test_cpp_host_layer(hip):
    assert os.path.exists(BIN), "tests/cpp/host_api_test is not built (run __graft_entry__.build())"
    out = subprocess.run([BIN], capture_output=True, text=True, timeout=90)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "ALL OK" in out.stdout
