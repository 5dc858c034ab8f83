"""Python mirror of the reference engine's static operator structs, running
on the gfx950 kernels through the C ABI.

Names and argument order follow source/CortexMind/framework/Engine/AVX2/:
inputs ``Xx``/``Xy``, output ``Xz``, sizes last (reduce.hpp:49-329,
broadcast.hpp:28-57, matrix.hpp:38-160).  Arguments are DeviceArrays; every
call is asynchronous on ``stream`` (None = null stream).  Where the
reference exits the process on an error (CXM_ASSERT,
Tools/Error/errors.cpp:14-23), these raise CxmError.
"""
from __future__ import annotations

import ctypes

import numpy as np

from ._lib import (ACT_EXP, ACT_NONE, ACT_RELU, ACT_SIGMOID, ACT_TANH, FN_ABS, FN_COS, FN_ERF,
                   FN_EXP, FN_INVERSE, FN_LOG, FN_NEG, FN_RCP, FN_RSQRT, FN_SIGN, FN_SIN, FN_SQRT,
                   FN_SQUARE, OP_ADD, OP_DIV, OP_MAX, OP_MIN, OP_MUL, OP_POW, OP_SUB, call)

__all__ = ["reduce", "Broadcast", "matrix_t", "ScalarOp", "wise", "activation", "softmax", "gemm",
           "train", "Mlp3", "ACT_NONE", "ACT_RELU", "ACT_SIGMOID", "ACT_TANH", "ACT_EXP"]


def _p(a):
    return None if a is None else a.ptr


def _s(stream):
    return stream.handle if stream is not None else None


class reduce:
    """avx2::reduce (Engine/AVX2/reduce.hpp:35-330): flat (Xx, Xz, N) and
    axis (Xx, Xz, outer, dim, inner) forms."""

    @staticmethod
    def _run(op, Xx, Xz, sizes, stream):
        if len(sizes) == 1:
            call(f"cxm_reduce_{op}_flat_f32", _p(Xx), _p(Xz), sizes[0], _s(stream))
        else:
            outer, dim, inner = sizes
            call(f"cxm_reduce_{op}_f32", _p(Xx), _p(Xz), outer, dim, inner, _s(stream))

    @staticmethod
    def sum(Xx, Xz, *sizes, stream=None):
        reduce._run("sum", Xx, Xz, sizes, stream)

    @staticmethod
    def mean(Xx, Xz, *sizes, stream=None):
        reduce._run("mean", Xx, Xz, sizes, stream)

    @staticmethod
    def max(Xx, Xz, *sizes, stream=None):
        reduce._run("max", Xx, Xz, sizes, stream)

    @staticmethod
    def argmax(Xx, Xz, *sizes, stream=None):
        reduce._run("argmax", Xx, Xz, sizes, stream)

    @staticmethod
    def min(Xx, Xz, *sizes, stream=None):
        reduce._run("min", Xx, Xz, sizes, stream)

    @staticmethod
    def argmin(Xx, Xz, *sizes, stream=None):
        reduce._run("argmin", Xx, Xz, sizes, stream)

    @staticmethod
    def norm1(Xx, Xz, *sizes, stream=None):
        reduce._run("norm1", Xx, Xz, sizes, stream)

    @staticmethod
    def norm2(Xx, Xz, *sizes, stream=None):
        reduce._run("norm2", Xx, Xz, sizes, stream)

    @staticmethod
    def var(Xx, Xz, *sizes, stream=None):
        reduce._run("var", Xx, Xz, sizes, stream)

    @staticmethod
    def stdv(Xx, Xz, *sizes, stream=None):
        reduce._run("stdv", Xx, Xz, sizes, stream)


class _BcastAxis:
    def __init__(self, fn):
        self._fn = fn

    def _run(self, op, Xx, Xy, Xz, M, N, stream):
        call(self._fn, _p(Xx), _p(Xy), _p(Xz), M, N, op, _s(stream))

    # out-of-place (Xx, Xy, Xz, M, N); in-place (Xx, Xy, M, N) writes Xx
    def _dispatch(self, op, args, stream):
        if len(args) == 5:
            Xx, Xy, Xz, M, N = args
        else:
            Xx, Xy, M, N = args
            Xz = Xx
        self._run(op, Xx, Xy, Xz, M, N, stream)

    def add(self, *args, stream=None):
        self._dispatch(OP_ADD, args, stream)

    def sub(self, *args, stream=None):
        self._dispatch(OP_SUB, args, stream)

    def mul(self, *args, stream=None):
        self._dispatch(OP_MUL, args, stream)

    def div(self, *args, stream=None):
        self._dispatch(OP_DIV, args, stream)


class Broadcast:
    """avx2::Broadcast::row / ::col (Engine/AVX2/broadcast.hpp:20-57)."""

    row = _BcastAxis("cxm_bcast_row_f32")
    col = _BcastAxis("cxm_bcast_col_f32")


class matrix_t:
    """avx2::matrix_t (Engine/AVX2/matrix.hpp:38-160) / nv::Matrix
    (Engine/CUDA/matrix.cuh:11-26)."""

    @staticmethod
    def _bin(op, args, stream):
        if len(args) == 4:
            Xx, Xy, Xz, N = args
        else:
            Xx, Xy, N = args
            Xz = Xx
        call("cxm_binary_f32", _p(Xx), _p(Xy), _p(Xz), N, op, _s(stream))

    @staticmethod
    def add(*args, stream=None):
        matrix_t._bin(OP_ADD, args, stream)

    @staticmethod
    def sub(*args, stream=None):
        matrix_t._bin(OP_SUB, args, stream)

    @staticmethod
    def mul(*args, stream=None):
        matrix_t._bin(OP_MUL, args, stream)

    @staticmethod
    def div(*args, stream=None):
        matrix_t._bin(OP_DIV, args, stream)

    @staticmethod
    def max(*args, stream=None):
        matrix_t._bin(OP_MAX, args, stream)

    @staticmethod
    def min(*args, stream=None):
        matrix_t._bin(OP_MIN, args, stream)

    @staticmethod
    def matmul(Xx, Xy, Xz, xN, yN, zN, stream=None):
        """Row-major Xz[xN, zN] = Xx[xN, yN] * Xy[yN, zN] (matrix.hpp:119)."""
        call("cxm_matmul_f32", _p(Xx), _p(Xy), _p(Xz), xN, yN, zN, _s(stream))

    @staticmethod
    def matmul_t(Xx, Xy, Xz, xN, yN, zN, dtype, stream=None):
        """matmul for a CXM_DT_* dtype: nv::Matrix::matmul's bf16 / fp16
        branches (Engine/CUDA/matrix.cu:112-159) on 16-bit element arrays,
        fp32 accumulation, one rounding to the 16-bit output."""
        call("cxm_matmul_t", _p(Xx), _p(Xy), _p(Xz), xN, yN, zN, dtype, _s(stream))


class ScalarOp:
    """avx2::ScalarOp (Engine/AVX2/scalar.cpp:89-119): Xz = Xx op value."""

    @staticmethod
    def _run(op, Xx, value, Xz, N, stream):
        call("cxm_scalar_f32", _p(Xx), float(value), _p(Xz), N, op, _s(stream))

    @staticmethod
    def add(Xx, value, Xz, N, stream=None):
        ScalarOp._run(OP_ADD, Xx, value, Xz, N, stream)

    @staticmethod
    def sub(Xx, value, Xz, N, stream=None):
        ScalarOp._run(OP_SUB, Xx, value, Xz, N, stream)

    @staticmethod
    def mul(Xx, value, Xz, N, stream=None):
        ScalarOp._run(OP_MUL, Xx, value, Xz, N, stream)

    @staticmethod
    def div(Xx, value, Xz, N, stream=None):
        ScalarOp._run(OP_DIV, Xx, value, Xz, N, stream)


class wise:
    """avx2::wise / nv::ElementWise (Engine/AVX2/wise.hpp:28-42,
    Engine/CUDA/element_wise.cuh:11-27): Xz = fn(Xx) over N elements (N
    defaults to Xx.size, the TensorView's element count)."""

    @staticmethod
    def _fn(fn, Xx, Xz, N, stream):
        call("cxm_wise_f32", _p(Xx), _p(Xz), Xx.size if N is None else N, fn, _s(stream))

    @staticmethod
    def square(Xx, Xz, N=None, stream=None):
        wise._fn(FN_SQUARE, Xx, Xz, N, stream)

    @staticmethod
    def sqrt(Xx, Xz, N=None, stream=None):
        wise._fn(FN_SQRT, Xx, Xz, N, stream)

    @staticmethod
    def rsqrt(Xx, Xz, N=None, stream=None):
        wise._fn(FN_RSQRT, Xx, Xz, N, stream)

    @staticmethod
    def log(Xx, Xz, N=None, stream=None):
        wise._fn(FN_LOG, Xx, Xz, N, stream)

    @staticmethod
    def exp(Xx, Xz, N=None, stream=None):
        wise._fn(FN_EXP, Xx, Xz, N, stream)

    @staticmethod
    def erf(Xx, Xz, N=None, stream=None):
        wise._fn(FN_ERF, Xx, Xz, N, stream)

    @staticmethod
    def sin(Xx, Xz, N=None, stream=None):
        wise._fn(FN_SIN, Xx, Xz, N, stream)

    @staticmethod
    def cos(Xx, Xz, N=None, stream=None):
        wise._fn(FN_COS, Xx, Xz, N, stream)

    @staticmethod
    def abs(Xx, Xz, N=None, stream=None):
        wise._fn(FN_ABS, Xx, Xz, N, stream)

    @staticmethod
    def neg(Xx, Xz, N=None, stream=None):
        wise._fn(FN_NEG, Xx, Xz, N, stream)

    @staticmethod
    def rcp(Xx, Xz, N=None, stream=None):
        wise._fn(FN_RCP, Xx, Xz, N, stream)

    @staticmethod
    def inverse(Xx, Xz, N=None, stream=None):
        wise._fn(FN_INVERSE, Xx, Xz, N, stream)

    @staticmethod
    def sign(Xx, Xz, N=None, stream=None):
        wise._fn(FN_SIGN, Xx, Xz, N, stream)

    @staticmethod
    def pow(Xx, y, Xz, N=None, stream=None):
        """pow(Xx, value) when y is a number, else elementwise pow(Xx, Xy)."""
        n = Xx.size if N is None else N
        if isinstance(y, (int, float)):
            call("cxm_scalar_f32", _p(Xx), float(y), _p(Xz), n, OP_POW, _s(stream))
        else:
            call("cxm_binary_f32", _p(Xx), _p(y), _p(Xz), n, OP_POW, _s(stream))

    @staticmethod
    def lerp(Xx, value1, value2, Xz, N, stream=None):
        call("cxm_lerp_f32", _p(Xx), float(value1), float(value2), _p(Xz), N, _s(stream))

    @staticmethod
    def clamp(Xx, lo, hi, Xz, N, stream=None):
        call("cxm_clamp_f32", _p(Xx), float(lo), float(hi), _p(Xz), N, _s(stream))

    @staticmethod
    def gather(Xx, Xy, Xz, N, x_n=None, stream=None):
        """Xz[i] = Xx[Xy[i]]; Xx's dtype (float32 or int32) picks the form."""
        xn = Xx.size if x_n is None else x_n
        fn = "cxm_gather_i32" if np.dtype(Xx.dtype) == np.int32 else "cxm_gather_f32"
        call(fn, _p(Xx), xn, _p(Xy), _p(Xz), N, _s(stream))


class activation:
    """Tensor-level relu / sigmoid / tanh / exp (Engine/AVX2/functions.hpp:
    186-188, 372-374, 381-383, 405-411), plus the fused affine forms."""

    @staticmethod
    def apply(Xx, Xz, N, act, stream=None):
        call("cxm_unary_f32", _p(Xx), _p(Xz), N, act, _s(stream))

    @staticmethod
    def affine_fwd(X, scale, bias, Y, M, N, act, stream=None):
        call("cxm_affine_act_fwd_f32", _p(X), _p(scale), _p(bias), _p(Y), M, N, act, _s(stream))

    @staticmethod
    def affine_bwd(X, scale, Y, dY, dX, dscale, dbias, M, N, act, stream=None):
        call("cxm_affine_act_bwd_f32", _p(X), _p(scale), _p(Y), _p(dY), _p(dX), _p(dscale),
             _p(dbias), M, N, act, _s(stream))


class softmax:
    """Row softmax / log-softmax over the last axis, forward and backward."""

    @staticmethod
    def forward(X, Y, rows, cols, log=False, stream=None):
        call("cxm_softmax_fwd_f32", _p(X), _p(Y), rows, cols, int(bool(log)), _s(stream))

    @staticmethod
    def backward(Y, dY, dX, rows, cols, log=False, stream=None):
        call("cxm_softmax_bwd_f32", _p(Y), _p(dY), _p(dX), rows, cols, int(bool(log)), _s(stream))


def gemm(A, B, C, m, k, n, trans_a=False, trans_b=False, bias=None, act=ACT_NONE, gate=None,
         stream=None):
    """C[m,n] = op(A) op(B) (+bias, act, relu-gate); see cxm_gemm_f32."""
    call("cxm_gemm_f32", _p(A), _p(B), _p(C), m, k, n, int(trans_a), int(trans_b), _p(bias),
         act, _p(gate), _s(stream))


class train:
    """Loss and optimizer pieces of the MLP step."""

    @staticmethod
    def softmax_xent(logits, labels, loss, dlogits, b, c, stream=None):
        call("cxm_softmax_xent_f32", _p(logits), _p(labels), _p(loss), _p(dlogits), b, c,
             _s(stream))

    @staticmethod
    def sgd(W, G, lr, N, stream=None):
        call("cxm_sgd_f32", _p(W), _p(G), float(lr), N, _s(stream))


class Mlp3:
    """The 3-layer ReLU MLP training step (cxm_mlp3_*): owns the activation
    and gradient buffers; parameters are caller-owned DeviceArrays
    {w1, b1, w2, b2, w3, b3}, updated in place by each step."""

    def __init__(self, batch, d0, d1, d2, d3):
        self.dims = (batch, d0, d1, d2, d3)
        self._h = ctypes.c_void_p(None)
        call("cxm_mlp3_create", ctypes.byref(self._h), batch, d0, d1, d2, d3)

    def step(self, x, labels, params, lr, loss, stream=None):
        call("cxm_mlp3_step_f32", self._h, _p(x), _p(labels), _p(params["w1"]), _p(params["b1"]),
             _p(params["w2"]), _p(params["b2"]), _p(params["w3"]), _p(params["b3"]), float(lr),
             _p(loss), _s(stream))

    def last_side(self):
        """Side workgroups of the last step's paired weight-gradient launch
        (0: the output layer's finish and the b1 step ran as kernels)."""
        n = ctypes.c_uint(0)
        call("cxm_mlp3_last_side", self._h, ctypes.byref(n))
        return n.value

    def close(self):
        if self._h.value:
            call("cxm_mlp3_destroy", self._h)
            self._h = ctypes.c_void_p(None)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
