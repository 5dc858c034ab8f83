"""The C++ host layers end to end on the GPU, built by __graft_entry__.build()
with g++ against the in-tree library:
  * tests/cpp/host_api_test (include/cortex_hip.hpp) checks reduce /
    Broadcast / matrix_t / wise / activation results against values it
    computes itself (exact integers);
  * tests/cpp/nv_api_test (include/cortex_hip_nv.hpp) drives nv::ElementWise
    / Matrix / ScalarKernel over TensorView in fp32, bf16 and fp16 (exact
    small integers), including matmul's shape inference;
  * tests/cpp/graph_test (include/cortex_hip_graph.hpp) checks Storage /
    Tensor::to / the caching pool, that three SGD steps of the MLP through
    the GradientFlow graph agree with cxm_mlp3_step_f32 (losses within 1e-5
    relative, parameters within 1e-4 of their weight scale), and
    gradient accumulation over two consumers."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "host_api_test")
GRAPH = os.path.join(HERE, "cpp", "graph_test")
NV = os.path.join(HERE, "cpp", "nv_api_test")

pytestmark = pytest.mark.gpu


def test_cpp_host_layer(hip):
    assert os.path.exists(BIN), "tests/cpp/host_api_test is not built (run __graft_entry__.build())"
    out = subprocess.run([BIN], capture_output=True, text=True, timeout=90)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "ALL OK" in out.stdout


def test_cpp_graph_storage_pool(hip):
    assert os.path.exists(GRAPH), "tests/cpp/graph_test is not built (run __graft_entry__.build())"
    out = subprocess.run([GRAPH], capture_output=True, text=True, timeout=110)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "ALL OK" in out.stdout


def test_cpp_nv_operator_api(hip):
    assert os.path.exists(NV), "tests/cpp/nv_api_test is not built (run __graft_entry__.build())"
    out = subprocess.run([NV], capture_output=True, text=True, timeout=90)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "ALL OK" in out.stdout
