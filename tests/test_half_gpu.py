"""bf16 / fp16: the dtype conversions (Tools/cast.cpp:7-90) and the 16-bit
forms of the elementwise surface, against the oracle (which restates
convert() and computes the op in fp32 between two conversions, as the
reference's kernel_t does, Engine/AVX2/wise.cpp:17-52).

Bars: conversions bit-exact (exhaustive over the 65536 16-bit patterns,
NaN compared as NaN); + - * / max min, ReLU and the exact math functions
bit-exact; transcendentals (sigmoid, tanh, exp, log, sin, cos, erf, rsqrt,
pow) within 1 unit of the 16-bit type, since the fp32 value they round
from is itself within 2 fp32 ulp.
"""
import numpy as np
import pytest

from cortexmind_amd._lib import (ACT_EXP, ACT_RELU, ACT_SIGMOID, ACT_TANH, DT_BF16, DT_F16, DT_F32, FN_ABS,
                                 FN_COS, FN_ERF, FN_EXP, FN_INVERSE, FN_LOG, FN_NEG, FN_RCP, FN_RSQRT, FN_SIGN,
                                 FN_SIN, FN_SQRT, FN_SQUARE, OP_ADD, OP_DIV, OP_MAX, OP_MIN, OP_MUL, OP_POW, OP_SUB,
                                 E_INVALID, call, lib)
from cortexmind_amd.data import SplitMix64

from gpu_util import dev, empty

pytestmark = pytest.mark.gpu

DTS = [DT_BF16, DT_F16]


def to16(f32, dt, orc):
    return orc.convert(np.ascontiguousarray(f32, np.float32), DT_F32, dt)


def same16(a, b, dt, orc, ulps=0):
    """16-bit patterns equal (NaN == NaN), or within `ulps` units of the type."""
    fa = orc.convert(a, dt, DT_F32).astype(np.float64)
    fb = orc.convert(b, dt, DT_F32).astype(np.float64)
    na, nb = np.isnan(fa), np.isnan(fb)
    if not np.array_equal(na, nb):
        return False
    a, b = a[~na].astype(np.int64), b[~na].astype(np.int64)
    if ulps == 0:
        return np.array_equal(a, b)
    # ordered integer distance of the sign-magnitude patterns
    oa = np.where(a & 0x8000, -(a & 0x7FFF), a)
    ob = np.where(b & 0x8000, -(b & 0x7FFF), b)
    return int(np.abs(oa - ob).max(initial=0)) <= ulps


def gpu_convert(src, sdt, ddt, off=0):
    n = src.size
    d_src = dev(src, off) if src.dtype == np.float32 else _dev16(src, off)
    if ddt == DT_F32:
        d_dst = empty((n,), np.float32, offset_floats=off)
    else:
        d_dst = _empty16(n, off)
    call("cxm_convert", d_dst.ptr, ddt, d_src.ptr, sdt, n, None)
    return d_dst.numpy()


def _dev16(a, off=0):
    return dev(np.ascontiguousarray(a, np.uint16), off)  # off counts 16-bit elements


def _empty16(n, off=0):
    return _dev16(np.zeros(n, np.uint16), off)


@pytest.mark.parametrize("dt", DTS)
def test_widen_exhaustive(hip, orc, dt):
    h = np.arange(65536, dtype=np.uint16)
    got = gpu_convert(h, dt, DT_F32)
    ref = orc.convert(h, dt, DT_F32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("n,off", [(1, 0), (9, 0), (100003, 0), (4099, 1)])
def test_narrow(hip, orc, dt, n, off):
    g = SplitMix64(900 + n + dt)
    f = g.normal((n,), 0.0, 50.0)
    sp = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65520.0, 3.4e38, 1e-40, 6e-8, 1.00390625], np.float32)
    f[: min(n, sp.size)] = sp[: min(n, sp.size)]
    got = gpu_convert(f, DT_F32, dt, off)
    assert same16(got, orc.convert(f, DT_F32, dt), dt, orc)


def test_16_to_16(hip, orc):
    h = np.arange(0, 65536, 7, dtype=np.uint16)
    for s, d in [(DT_BF16, DT_F16), (DT_F16, DT_BF16)]:
        got = gpu_convert(h, s, d)
        ref = orc.convert(orc.convert(h, s, DT_F32), DT_F32, d)
        assert same16(got, ref, d, orc)


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("op", [OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_MAX, OP_MIN, OP_POW])
@pytest.mark.parametrize("n,off", [(7, 0), (100003, 0), (1031, 1)])
def test_binary_scalar(hip, orc, dt, op, n, off):
    g = SplitMix64(1000 + 10 * op + n + dt)
    lo = 0.1 if op == OP_POW else -20.0
    x = to16(g.uniform((n,), lo, 20.0), dt, orc)
    y = to16(g.uniform((n,), -3.0 if op == OP_POW else -20.0, 3.0 if op == OP_POW else 20.0), dt, orc)
    dx, dy, dz = _dev16(x, off), _dev16(y, off), _empty16(n, off)
    call("cxm_binary_t", dx.ptr, dy.ptr, dz.ptr, n, op, dt, None)
    ulps = 1 if op == OP_POW else 0
    assert same16(dz.numpy(), orc.binary_t(x, y, op, dt), dt, orc, ulps)
    call("cxm_scalar_t", dx.ptr, np.float32(1.37), dz.ptr, n, op, dt, None)
    assert same16(dz.numpy(), orc.scalar_t(x, 1.37, op, dt), dt, orc, ulps)


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("act", [ACT_RELU, ACT_SIGMOID, ACT_TANH, ACT_EXP])
def test_activations(hip, orc, dt, act):
    n = 100003
    x = to16(SplitMix64(1100 + act + dt).normal((n,), 0.0, 3.0), dt, orc)
    dx, dz = _dev16(x), _empty16(n)
    call("cxm_unary_t", dx.ptr, dz.ptr, n, act, dt, None)
    assert same16(dz.numpy(), orc.unary_t(x, act, dt), dt, orc, 0 if act == ACT_RELU else 1)


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("fn", [FN_SQUARE, FN_SQRT, FN_RSQRT, FN_LOG, FN_EXP, FN_ERF, FN_SIN, FN_COS, FN_ABS, FN_NEG,
                                FN_RCP, FN_INVERSE, FN_SIGN])
def test_wise(hip, orc, dt, fn):
    n = 50001
    g = SplitMix64(1200 + fn + dt)
    x = g.uniform((n,), 0.01, 30.0) if fn in (FN_SQRT, FN_RSQRT, FN_LOG) else g.normal((n,), 0.0, 4.0)
    x = to16(x, dt, orc)
    dx, dz = _dev16(x), _empty16(n)
    call("cxm_wise_t", dx.ptr, dz.ptr, n, fn, dt, None)
    exact = fn in (FN_SQUARE, FN_SQRT, FN_ABS, FN_NEG, FN_RCP, FN_INVERSE, FN_SIGN)
    assert same16(dz.numpy(), orc.wise_t(x, fn, dt), dt, orc, 0 if exact else 1)


def test_f32_forwarding_and_errors(hip, orc):
    x = SplitMix64(5).normal((1000,))
    dx, dz = dev(x), empty((1000,))
    call("cxm_wise_t", dx.ptr, dz.ptr, 1000, FN_SQUARE, DT_F32, None)
    assert np.array_equal(dz.numpy(), orc.wise(x, FN_SQUARE))
    assert lib().cxm_convert(dz.ptr, 7, dx.ptr, DT_F32, 10, None) == E_INVALID
    assert lib().cxm_binary_t(dx.ptr, dx.ptr, dz.ptr, 10, 9, DT_BF16, None) == E_INVALID
    assert lib().cxm_wise_t(dx.ptr, dz.ptr, 10, 0, 5, None) == E_INVALID
