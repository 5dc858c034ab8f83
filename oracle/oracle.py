"""ctypes front end of the CPU oracle (oracle/cxm_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU baseline,
never as part of the product path.  Each wrapper takes and returns numpy
arrays; the C function it calls cites the reference lines it restates.

Parity pins of each oracle function (the checks that would catch a dropped
term, a wrong fold order or a transposed operand) live in
tests/test_oracle.py; every function below is covered there.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libcxm_oracle.so")

ADD, SUB, MUL, DIV, MAX, MIN, POW = range(7)
DT_F32, DT_BF16, DT_F16 = range(3)
(FN_SQUARE, FN_SQRT, FN_RSQRT, FN_LOG, FN_EXP, FN_ERF, FN_SIN, FN_COS, FN_ABS, FN_NEG, FN_RCP,
 FN_INVERSE, FN_SIGN) = range(13)
ACT_NONE, ACT_RELU, ACT_SIGMOID, ACT_TANH, ACT_EXP = range(5)

_F = ctypes.POINTER(ctypes.c_float)
_I = ctypes.POINTER(ctypes.c_int32)
_SZ = ctypes.c_size_t

_lib = None


def build() -> str:
    """Compile the oracle with its Makefile (gcc only)."""
    import subprocess

    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        l = ctypes.CDLL(_LIB_PATH)
        sigs = {
            "orc_reduce_sum_flat": [_F, _F, _SZ],
            "orc_reduce_sum": [_F, _F, _SZ, _SZ, _SZ],
            "orc_reduce_mean_flat": [_F, _F, _SZ],
            "orc_reduce_mean": [_F, _F, _SZ, _SZ, _SZ],
            "orc_reduce_max_flat": [_F, _F, _SZ],
            "orc_reduce_max": [_F, _F, _SZ, _SZ, _SZ],
            "orc_reduce_argmax_flat": [_F, _I, _SZ],
            "orc_reduce_argmax": [_F, _I, _SZ, _SZ, _SZ],
            "orc_reduce_argmin_flat": [_F, _I, _SZ],
            "orc_reduce_argmin": [_F, _I, _SZ, _SZ, _SZ],
            **{f"orc_reduce_{op}_flat": [_F, _F, _SZ] for op in ("min", "norm1", "norm2", "var", "stdv")},
            **{f"orc_reduce_{op}": [_F, _F, _SZ, _SZ, _SZ] for op in ("min", "norm1", "norm2", "var", "stdv")},
            "orc_binary": [_F, _F, _F, _SZ, ctypes.c_int],
            "orc_bcast_row": [_F, _F, _F, _SZ, _SZ, ctypes.c_int],
            "orc_bcast_col": [_F, _F, _F, _SZ, _SZ, ctypes.c_int],
            "orc_scalar": [_F, ctypes.c_float, _F, _SZ, ctypes.c_int],
            "orc_unary": [_F, _F, _SZ, ctypes.c_int],
            "orc_wise": [_F, _F, _SZ, ctypes.c_int],
            "orc_convert": [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, _SZ],
            "orc_act_bwd": [_F, _F, _F, _SZ, ctypes.c_int],
            "orc_lerp": [_F, ctypes.c_float, ctypes.c_float, _F, _SZ],
            "orc_clamp": [_F, ctypes.c_float, ctypes.c_float, _F, _SZ],
            "orc_gather_f32": [_F, _SZ, _I, _F, _SZ],
            "orc_gather_i32": [_I, _SZ, _I, _I, _SZ],
            "orc_affine_act_fwd": [_F, _F, _F, _F, _SZ, _SZ, ctypes.c_int],
            "orc_affine_act_bwd": [_F, _F, _F, _F, _F, _F, _F, _SZ, _SZ, ctypes.c_int],
            "orc_softmax_fwd": [_F, _F, _SZ, _SZ, ctypes.c_int],
            "orc_softmax_bwd": [_F, _F, _F, _SZ, _SZ, ctypes.c_int],
            "orc_matmul": [_F, _F, _F, _SZ, _SZ, _SZ],
            "orc_gemm": [_F, _F, _F, _SZ, _SZ, _SZ, ctypes.c_int, ctypes.c_int],
            "orc_softmax_xent": [_F, _I, _F, _F, _SZ, _SZ],
            "orc_sgd": [_F, _F, ctypes.c_float, _SZ],
            "orc_mlp_step": [_F, _I, _F, _F, _F, _F, _F, _F, _SZ, _SZ, _SZ, _SZ, _SZ,
                             ctypes.c_float, _F],
        }
        for name, args in sigs.items():
            fn = getattr(l, name)
            fn.argtypes = args
            fn.restype = None
        _lib = l
    return _lib


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def _i(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(_I)


def _c32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ------------------------------------------------------------ reductions

def reduce_flat(op: str, x) -> np.ndarray:
    x = _c32(x).ravel()
    if op in ("argmax", "argmin"):
        z = np.zeros(1, np.int32)
        getattr(lib(), f"orc_reduce_{op}_flat")(_f(x), _i(z), x.size)
        return z
    z = np.zeros(1, np.float32)
    getattr(lib(), f"orc_reduce_{op}_flat")(_f(x), _f(z), x.size)
    return z


def reduce_axis(op: str, x, outer: int, dim: int, inner: int) -> np.ndarray:
    x = _c32(x).ravel()
    assert x.size == outer * dim * inner
    if op in ("argmax", "argmin"):
        z = np.zeros(outer * inner, np.int32)
        getattr(lib(), f"orc_reduce_{op}")(_f(x), _i(z), outer, dim, inner)
        return z
    z = np.zeros(outer * inner, np.float32)
    getattr(lib(), f"orc_reduce_{op}")(_f(x), _f(z), outer, dim, inner)
    return z


# ----------------------------------------------------------- elementwise

def binary(x, y, op: int) -> np.ndarray:
    x, y = _c32(x), _c32(y)
    z = np.empty_like(x)
    lib().orc_binary(_f(x), _f(y), _f(z), x.size, op)
    return z


def bcast_row(x, y, op: int) -> np.ndarray:
    x, y = _c32(x), _c32(y)
    m, n = x.shape
    z = np.empty_like(x)
    lib().orc_bcast_row(_f(x), _f(y), _f(z), m, n, op)
    return z


def bcast_col(x, y, op: int) -> np.ndarray:
    x, y = _c32(x), _c32(y)
    m, n = x.shape
    z = np.empty_like(x)
    lib().orc_bcast_col(_f(x), _f(y), _f(z), m, n, op)
    return z


def scalar(x, value: float, op: int) -> np.ndarray:
    x = _c32(x)
    z = np.empty_like(x)
    lib().orc_scalar(_f(x), float(value), _f(z), x.size, op)
    return z


def unary(x, act: int) -> np.ndarray:
    x = _c32(x)
    z = np.empty_like(x)
    lib().orc_unary(_f(x), _f(z), x.size, act)
    return z


def wise(x, fn: int) -> np.ndarray:
    x = _c32(x)
    z = np.empty_like(x)
    lib().orc_wise(_f(x), _f(z), x.size, fn)
    return z


def convert(src, src_dt: int, dst_dt: int) -> np.ndarray:
    """Tools/cast.cpp convert(): float32 <-> bf16/f16 (16-bit data as uint16)."""
    src = np.ascontiguousarray(src, dtype=np.float32 if src_dt == DT_F32 else np.uint16)
    dst = np.empty(src.shape, np.float32 if dst_dt == DT_F32 else np.uint16)
    lib().orc_convert(dst.ctypes.data, dst_dt, src.ctypes.data, src_dt, src.size)
    return dst


def binary_t(x, y, op: int, dt: int) -> np.ndarray:
    """16-bit binary op: widen, fp32 op, round once (wise.cpp:17-52 kernel_t)."""
    return convert(binary(convert(x, dt, DT_F32), convert(y, dt, DT_F32), op), DT_F32, dt)


def scalar_t(x, value: float, op: int, dt: int) -> np.ndarray:
    v = convert(convert(np.array([value], np.float32), DT_F32, dt), dt, DT_F32)[0]
    return convert(scalar(convert(x, dt, DT_F32), v, op), DT_F32, dt)


def unary_t(x, act: int, dt: int) -> np.ndarray:
    return convert(unary(convert(x, dt, DT_F32), act), DT_F32, dt)


def wise_t(x, fn: int, dt: int) -> np.ndarray:
    return convert(wise(convert(x, dt, DT_F32), fn), DT_F32, dt)


def act_bwd(y, dy, act: int) -> np.ndarray:
    y, dy = _c32(y), _c32(dy)
    dx = np.empty_like(y)
    lib().orc_act_bwd(_f(y), _f(dy), _f(dx), y.size, act)
    return dx


def lerp(x, v1: float, v2: float) -> np.ndarray:
    x = _c32(x)
    z = np.empty_like(x)
    lib().orc_lerp(_f(x), float(v1), float(v2), _f(z), x.size)
    return z


def clamp(x, lo: float, hi: float) -> np.ndarray:
    x = _c32(x)
    z = np.empty_like(x)
    lib().orc_clamp(_f(x), float(lo), float(hi), _f(z), x.size)
    return z


def gather(x, idx) -> np.ndarray:
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    if np.asarray(x).dtype == np.int32:
        x = np.ascontiguousarray(x, dtype=np.int32)
        z = np.empty(idx.size, np.int32)
        lib().orc_gather_i32(_i(x), x.size, _i(idx), _i(z), idx.size)
        return z
    x = _c32(x)
    z = np.empty(idx.size, np.float32)
    lib().orc_gather_f32(_f(x), x.size, _i(idx), _f(z), idx.size)
    return z


def affine_act_fwd(x, scale, bias, act: int) -> np.ndarray:
    x, scale, bias = _c32(x), _c32(scale), _c32(bias)
    m, n = x.shape
    y = np.empty_like(x)
    lib().orc_affine_act_fwd(_f(x), _f(scale), _f(bias), _f(y), m, n, act)
    return y


def affine_act_bwd(x, scale, y, dy, act: int):
    x, scale, y, dy = _c32(x), _c32(scale), _c32(y), _c32(dy)
    m, n = x.shape
    dx = np.empty_like(x)
    ds = np.empty(n, np.float32)
    db = np.empty(n, np.float32)
    lib().orc_affine_act_bwd(_f(x), _f(scale), _f(y), _f(dy), _f(dx), _f(ds), _f(db), m, n, act)
    return dx, ds, db


# --------------------------------------------------------------- softmax

def softmax_fwd(x, log: bool = False) -> np.ndarray:
    x = _c32(x)
    rows, cols = x.shape
    y = np.empty_like(x)
    lib().orc_softmax_fwd(_f(x), _f(y), rows, cols, int(log))
    return y


def softmax_bwd(y, dy, log: bool = False) -> np.ndarray:
    y, dy = _c32(y), _c32(dy)
    rows, cols = y.shape
    dx = np.empty_like(y)
    lib().orc_softmax_bwd(_f(y), _f(dy), _f(dx), rows, cols, int(log))
    return dx


# ---------------------------------------------------------------- matmul

def matmul(a, b) -> np.ndarray:
    a, b = _c32(a), _c32(b)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().orc_matmul(_f(a), _f(b), _f(c), m, k, n)
    return c


def gemm(a, b, trans_a: bool = False, trans_b: bool = False) -> np.ndarray:
    a, b = _c32(a), _c32(b)
    m, k = (a.shape[1], a.shape[0]) if trans_a else a.shape
    n = b.shape[0] if trans_b else b.shape[1]
    c = np.empty((m, n), np.float32)
    lib().orc_gemm(_f(a), _f(b), _f(c), m, k, n, int(trans_a), int(trans_b))
    return c


# ------------------------------------------------------------------ MLP

def softmax_xent(logits, labels):
    logits = _c32(logits)
    labels = np.ascontiguousarray(labels, np.int32)
    b, c = logits.shape
    loss = np.zeros(1, np.float32)
    dl = np.empty_like(logits)
    lib().orc_softmax_xent(_f(logits), _i(labels), _f(loss), _f(dl), b, c)
    return float(loss[0]), dl


def sgd(w, g, lr: float) -> np.ndarray:
    w = _c32(w).copy()
    g = _c32(g)
    lib().orc_sgd(_f(w), _f(g), float(lr), w.size)
    return w


def mlp_step(x, labels, params: dict, lr: float) -> float:
    """One in-place SGD step on params {w1,b1,w2,b2,w3,b3}; returns the loss."""
    x = _c32(x)
    labels = np.ascontiguousarray(labels, np.int32)
    for k in params:
        assert params[k].dtype == np.float32 and params[k].flags.c_contiguous
    b, d0 = x.shape
    d1 = params["w1"].shape[1]
    d2 = params["w2"].shape[1]
    d3 = params["w3"].shape[1]
    loss = np.zeros(1, np.float32)
    lib().orc_mlp_step(_f(x), _i(labels), _f(params["w1"]), _f(params["b1"]), _f(params["w2"]),
                       _f(params["b2"]), _f(params["w3"]), _f(params["b3"]), b, d0, d1, d2, d3,
                       float(lr), _f(loss))
    return float(loss[0])
