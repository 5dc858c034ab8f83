"""CPU-only checks of the C ABI boundary: the library loads, exports every
function include/cxm_hip.h declares, and rejects bad arguments on the host
(before any HIP call, so these run without a GPU)."""
import ctypes
import numpy as np
import pytest

from cortexmind_amd import _lib


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    declared = _lib.header_symbols()
    assert len(declared) >= 40
    missing = [s for s in declared if not hasattr(lib, s)]
    assert missing == []
    # and the Python binding declares a signature for each of them
    unbound = [s for s in declared if s not in _lib.SIGNATURES and s != "cxm_error_string"]
    assert unbound == []


def test_library_carries_gfx950_device_code():
    data = open(_lib.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in data


def test_abi_header_is_plain_c():
    import re

    text = open(_lib.HEADER).read()
    code = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    assert re.findall(r"#include\s*<([^>]+)>", code) == ["stddef.h", "stdint.h"]
    for word in ("torch", "cuda", "hip_", "Tensor", "template", "class "):
        assert word not in code


def test_error_strings():
    lib = _lib.lib()
    assert lib.cxm_error_string(0) == b"success"
    assert b"invalid" in lib.cxm_error_string(_lib.E_INVALID)
    assert lib.cxm_error_string(-99) == b"unknown cxm status"


@pytest.mark.parametrize("fn,args", [
    ("cxm_reduce_sum_f32", (None, None, 4, 4, 1, None)),
    ("cxm_reduce_argmax_flat_f32", (None, None, 0, None)),
    ("cxm_binary_f32", (None, None, None, 4, 0, None)),
    ("cxm_bcast_row_f32", (None, None, None, 4, 4, 0, None)),
    ("cxm_scalar_f32", (None, 1.0, None, 4, 0, None)),
    ("cxm_unary_f32", (None, None, 4, 1, None)),
    ("cxm_affine_act_fwd_f32", (None, None, None, None, 4, 4, 1, None)),
    ("cxm_affine_act_bwd_f32", (None,) * 7 + (4, 4, 1, None)),
    ("cxm_softmax_fwd_f32", (None, None, 4, 4, 0, None)),
    ("cxm_softmax_bwd_f32", (None, None, None, 4, 4, 0, None)),
    ("cxm_gemm_f32", (None, None, None, 4, 4, 4, 0, 0, None, 0, None, None)),
    ("cxm_matmul_f32", (None, None, None, 4, 4, 4, None)),
    ("cxm_softmax_xent_f32", (None, None, None, None, 4, 4, None)),
    ("cxm_sgd_f32", (None, None, 0.1, 4, None)),
    ("cxm_mlp3_step_f32", (None,) * 9 + (0.1, None, None)),
])
def test_null_pointers_rejected_on_host(fn, args):
    assert getattr(_lib.lib(), fn)(*args) == _lib.E_INVALID


def test_bad_enums_rejected_on_host():
    lib = _lib.lib()
    p = ctypes.c_void_p(0x1000)  # never dereferenced: the enum check comes first
    assert lib.cxm_binary_f32(p, p, p, 4, 9, None) == _lib.E_INVALID
    assert lib.cxm_bcast_col_f32(p, p, p, 4, 4, _lib.OP_MAX, None) == _lib.E_INVALID
    assert lib.cxm_unary_f32(p, p, 4, 17, None) == _lib.E_INVALID
    assert lib.cxm_softmax_fwd_f32(p, p, 4, 4, 2, None) == _lib.E_INVALID
    assert lib.cxm_gemm_f32(p, p, p, 4, 4, 4, 0, 0, None, _lib.ACT_SIGMOID, None, None) == _lib.E_INVALID


def test_softmax_partial_overlap_rejected_on_host():
    """A softmax output that overlaps an input without being it is refused
    before any launch; exact in-place calls are accepted (run on the GPU in
    tests/test_softmax_gpu.py)."""
    lib = _lib.lib()
    x = ctypes.c_void_p(0x10000)
    y = ctypes.c_void_p(0x10000 + 16)  # one float4 into x's 4x64 floats
    assert lib.cxm_softmax_fwd_f32(x, y, 4, 64, 0, None) == _lib.E_INVALID
    assert lib.cxm_softmax_fwd_f32(y, x, 4, 64, 1, None) == _lib.E_INVALID
    far = ctypes.c_void_p(0x10000 + 4 * 4 * 64 * 2)
    assert lib.cxm_softmax_bwd_f32(x, far, y, 4, 64, 0, None) == _lib.E_INVALID
    assert lib.cxm_softmax_bwd_f32(far, x, y, 4, 64, 1, None) == _lib.E_INVALID


def test_empty_outputs_are_noops():
    lib = _lib.lib()
    p = ctypes.c_void_p(0x1000)
    assert lib.cxm_reduce_sum_f32(p, p, 0, 5, 3, None) == 0
    assert lib.cxm_binary_f32(p, p, p, 0, 0, None) == 0
    assert lib.cxm_softmax_fwd_f32(p, p, 0, 8, 0, None) == 0
    assert lib.cxm_gemm_f32(p, p, p, 0, 4, 4, 0, 0, None, 0, None, None) == 0


def test_cpp_host_layer_builds_and_links():
    """The C++ mirror header compiles with a plain host compiler and the
    test program links against the library (run on the GPU elsewhere)."""
    import os
    import subprocess

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    out = subprocess.run(["make", "-s", "-C", os.path.join(root, "tests", "cpp")], capture_output=True,
                         text=True)
    assert out.returncode == 0, out.stderr
    assert os.path.exists(os.path.join(root, "tests", "cpp", "host_api_test"))
    assert os.path.exists(os.path.join(root, "tests", "cpp", "graph_test"))
    assert os.path.exists(os.path.join(root, "tests", "cpp", "nv_api_test"))


def test_pool_core_bookkeeping():
    """The caching pool's bookkeeping (cortexmind_amd/csrc/pool.hpp) over a
    host backend, built with AddressSanitizer/UBSan: size classes, same-stream
    reuse, no cross-stream reuse, foreign/double frees, release-and-retry on
    out-of-memory, stream teardown, no leaks."""
    import os
    import subprocess

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    out = subprocess.run(["make", "-s", "-C", os.path.join(root, "tests", "cpp")], capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
    run = subprocess.run([os.path.join(root, "tests", "cpp", "pool_core_test")], capture_output=True, text=True,
                         timeout=60)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "ALL OK" in run.stdout


def test_timeline_build_exports_its_reader():
    """The diagnostics build (reduce.hip, softmax.hip, gemm.hip and mlp.hip with
    -DCXM_TIMELINE, built beside the library) carries gfx950 code and exports
    its table readers; the library itself does not."""
    import os

    path = os.path.join(os.path.dirname(_lib.LIB_PATH), "libcxm_hip_timeline.so")
    if not os.path.exists(path):
        pytest.skip("diagnostics build not built (make -C cortexmind_amd/csrc timeline)")
    tl = ctypes.CDLL(path)
    for name in ("cxm_timeline_read", "cxm_timeline_softmax_read", "cxm_timeline_gemm_read", "cxm_timeline_head_read"):
        assert hasattr(tl, name), name
    assert b"amdgcn-amd-amdhsa--gfx950" in open(path, "rb").read()
    assert not any(hasattr(_lib.lib(), n) for n in ("cxm_timeline_read", "cxm_timeline_softmax_read",
                                                    "cxm_timeline_gemm_read", "cxm_timeline_head_read"))
