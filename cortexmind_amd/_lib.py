"""ctypes binding of libcxm_hip.so, the C ABI declared in include/cxm_hip.h.

Loading never builds anything and never falls back to another code path: if
the library is missing the import fails loudly (build it with
``python -c "import __graft_entry__ as g; g.build()"`` or
``make -C cortexmind_amd/csrc``).  Loading the library does not touch the
GPU; the first HIP call does.
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcxm_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "cxm_hip.h")

OK = 0
E_INVALID = -1
E_TOO_LARGE = -2
E_NO_DEVICE = -3
E_CAPTURE = -4

OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_MAX, OP_MIN, OP_POW = range(7)
DT_F32, DT_BF16, DT_F16 = range(3)
(FN_SQUARE, FN_SQRT, FN_RSQRT, FN_LOG, FN_EXP, FN_ERF, FN_SIN, FN_COS, FN_ABS, FN_NEG, FN_RCP,
 FN_INVERSE, FN_SIGN) = range(13)
ACT_NONE, ACT_RELU, ACT_SIGMOID, ACT_TANH, ACT_EXP = range(5)

_P = ctypes.c_void_p  # device pointer, stream or event handle
_SZ = ctypes.c_size_t
_I = ctypes.c_int
_F = ctypes.c_float

class PoolStats(ctypes.Structure):
    """cxm_pool_stats_t."""
    _fields_ = [("bytes_in_use", ctypes.c_size_t), ("bytes_cached", ctypes.c_size_t),
                ("peak_in_use", ctypes.c_size_t), ("allocs", ctypes.c_uint64), ("hits", ctypes.c_uint64),
                ("frees", ctypes.c_uint64), ("device_allocs", ctypes.c_uint64)]


# name -> argtypes (every function returns int status)
SIGNATURES = {
    "cxm_device_count": [ctypes.POINTER(_I)],
    "cxm_set_device": [_I],
    "cxm_device_info": [ctypes.c_char_p, _SZ, ctypes.POINTER(_I), ctypes.c_char_p, _SZ],
    "cxm_device_sync": [],
    "cxm_dev_malloc": [ctypes.POINTER(_P), _SZ],
    "cxm_dev_free": [_P],
    "cxm_memcpy_h2d": [_P, _P, _SZ, _P],
    "cxm_memcpy_d2h": [_P, _P, _SZ, _P],
    "cxm_memcpy_d2d": [_P, _P, _SZ, _P],
    "cxm_memset": [_P, _I, _SZ, _P],
    "cxm_stream_create": [ctypes.POINTER(_P)],
    "cxm_stream_sync": [_P],
    "cxm_stream_destroy": [_P],
    "cxm_event_create": [ctypes.POINTER(_P)],
    "cxm_event_record": [_P, _P],
    "cxm_event_sync": [_P],
    "cxm_event_elapsed_ms": [ctypes.POINTER(_F), _P, _P],
    "cxm_event_destroy": [_P],
    "cxm_release_workspaces": [],
    "cxm_workspace_query": [_P, _I, ctypes.POINTER(_P), ctypes.POINTER(_SZ), ctypes.POINTER(_I)],
    "cxm_act_bwd_f32": [_P, _P, _P, _SZ, _I, _P],
    "cxm_convert": [_P, _I, _P, _I, _SZ, _P],
    "cxm_binary_t": [_P, _P, _P, _SZ, _I, _I, _P],
    "cxm_scalar_t": [_P, _F, _P, _SZ, _I, _I, _P],
    "cxm_unary_t": [_P, _P, _SZ, _I, _I, _P],
    "cxm_wise_t": [_P, _P, _SZ, _I, _I, _P],
    "cxm_pool_alloc": [ctypes.POINTER(_P), _SZ, _P],
    "cxm_pool_free": [_P],
    "cxm_pool_release": [],
    "cxm_pool_stats": [_P],
    "cxm_reduce_sum_flat_f32": [_P, _P, _SZ, _P],
    "cxm_reduce_mean_flat_f32": [_P, _P, _SZ, _P],
    "cxm_reduce_max_flat_f32": [_P, _P, _SZ, _P],
    "cxm_reduce_argmax_flat_f32": [_P, _P, _SZ, _P],
    "cxm_reduce_sum_f32": [_P, _P, _SZ, _SZ, _SZ, _P],
    "cxm_reduce_sum_noalloc_f32": [_P, _P, _SZ, _SZ, _SZ, _P],
    "cxm_reduce_mean_f32": [_P, _P, _SZ, _SZ, _SZ, _P],
    "cxm_reduce_max_f32": [_P, _P, _SZ, _SZ, _SZ, _P],
    "cxm_reduce_argmax_f32": [_P, _P, _SZ, _SZ, _SZ, _P],
    "cxm_reduce_min_flat_f32": [_P, _P, _SZ, _P],
    "cxm_reduce_min_f32": [_P, _P, _SZ, _SZ, _SZ, _P],
    "cxm_reduce_argmin_flat_f32": [_P, _P, _SZ, _P],
    "cxm_reduce_argmin_f32": [_P, _P, _SZ, _SZ, _SZ, _P],
    "cxm_reduce_norm1_flat_f32": [_P, _P, _SZ, _P],
    "cxm_reduce_norm1_f32": [_P, _P, _SZ, _SZ, _SZ, _P],
    "cxm_reduce_norm2_flat_f32": [_P, _P, _SZ, _P],
    "cxm_reduce_norm2_f32": [_P, _P, _SZ, _SZ, _SZ, _P],
    "cxm_reduce_var_flat_f32": [_P, _P, _SZ, _P],
    "cxm_reduce_var_f32": [_P, _P, _SZ, _SZ, _SZ, _P],
    "cxm_reduce_stdv_flat_f32": [_P, _P, _SZ, _P],
    "cxm_reduce_stdv_f32": [_P, _P, _SZ, _SZ, _SZ, _P],
    "cxm_binary_f32": [_P, _P, _P, _SZ, _I, _P],
    "cxm_bcast_row_f32": [_P, _P, _P, _SZ, _SZ, _I, _P],
    "cxm_bcast_col_f32": [_P, _P, _P, _SZ, _SZ, _I, _P],
    "cxm_scalar_f32": [_P, _F, _P, _SZ, _I, _P],
    "cxm_unary_f32": [_P, _P, _SZ, _I, _P],
    "cxm_wise_f32": [_P, _P, _SZ, _I, _P],
    "cxm_lerp_f32": [_P, _F, _F, _P, _SZ, _P],
    "cxm_clamp_f32": [_P, _F, _F, _P, _SZ, _P],
    "cxm_gather_f32": [_P, _SZ, _P, _P, _SZ, _P],
    "cxm_gather_i32": [_P, _SZ, _P, _P, _SZ, _P],
    "cxm_affine_act_fwd_f32": [_P, _P, _P, _P, _SZ, _SZ, _I, _P],
    "cxm_affine_act_bwd_f32": [_P, _P, _P, _P, _P, _P, _P, _SZ, _SZ, _I, _P],
    "cxm_softmax_fwd_f32": [_P, _P, _SZ, _SZ, _I, _P],
    "cxm_softmax_bwd_f32": [_P, _P, _P, _SZ, _SZ, _I, _P],
    "cxm_exchange_wait_limit": [ctypes.c_uint, _P],
    "cxm_softmax_stagger": [_I, _P],
    "cxm_matmul_f32": [_P, _P, _P, _SZ, _SZ, _SZ, _P],
    "cxm_gemm_f32": [_P, _P, _P, _SZ, _SZ, _SZ, _I, _I, _P, _I, _P, _P],
    "cxm_matmul_t": [_P, _P, _P, _SZ, _SZ, _SZ, _I, _P],
    "cxm_gemm_t": [_P, _P, _P, _SZ, _SZ, _SZ, _I, _I, _I, _P],
    "cxm_gemm16_kernel": [_I],
    "cxm_gemm_f32_kernel": [_I],
    "cxm_softmax_xent_f32": [_P, _P, _P, _P, _SZ, _SZ, _P],
    "cxm_sgd_f32": [_P, _P, _F, _SZ, _P],
    "cxm_reduce_sum_bwd_f32": [_P, _P, _SZ, _SZ, _SZ, _I, _P],
    "cxm_mlp3_last_side": [_P, ctypes.POINTER(ctypes.c_uint)],
    "cxm_mlp3_create": [ctypes.POINTER(_P), _SZ, _SZ, _SZ, _SZ, _SZ],
    "cxm_mlp3_step_f32": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _P, _P],
    "cxm_mlp3_destroy": [_P],
}


class CxmError(RuntimeError):
    def __init__(self, fn: str, status: int, text: str):
        super().__init__(f"{fn} failed: status {status} ({text})")
        self.status = status


def header_symbols(path: str = HEADER) -> list[str]:
    """Names of every function the C header declares."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cxm_\w+)\s*\(", text)))


_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library with argtypes set (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built; run make -C cortexmind_amd/csrc")
        l = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            if not hasattr(l, name):
                continue  # calling it raises AttributeError; build() checks completeness
            fn = getattr(l, name)
            fn.argtypes = args
            fn.restype = _I
        l.cxm_error_string.argtypes = [_I]
        l.cxm_error_string.restype = ctypes.c_char_p
        _lib = l
    return _lib


def check(fn: str, status: int) -> None:
    if status != OK:
        raise CxmError(fn, status, lib().cxm_error_string(status).decode())


def call(fn: str, *args) -> None:
    """Call an entry point and raise CxmError on a non-zero status."""
    check(fn, getattr(lib(), fn)(*args))
