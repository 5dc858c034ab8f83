"""Parity of the gfx950 elementwise math surface (cxm_wise_f32, pow, lerp,
clamp, gather) with the CPU oracle and float64.

Bars: square, abs, neg, sign, clamp, lerp (one fma rounding) and gather are
bit-exact with the oracle; sqrt and rcp/inverse are correctly rounded, so
bit-exact too; rsqrt, log, exp, erf, sin, cos and pow are within 2 ulp of
the float64 function rounded to float32.  Special values (0, -0, inf, NaN,
negative arguments of sqrt/log) give the IEEE results.  Inputs stay in the
normal range for the ulp bars: a denormal argument or result is an ulp
outlier by construction and is covered by the special-value checks instead.
"""
import numpy as np
import pytest
import scipy.special

from cortexmind_amd import engine
from cortexmind_amd._lib import (FN_ABS, FN_COS, FN_ERF, FN_EXP, FN_INVERSE, FN_LOG, FN_NEG,
                                 FN_RCP, FN_RSQRT, FN_SIGN, FN_SIN, FN_SQRT, FN_SQUARE, OP_POW,
                                 E_INVALID, call, lib)
from cortexmind_amd.data import SplitMix64

from gpu_util import dev, empty, ulp_dist

pytestmark = pytest.mark.gpu

SIZES = [(1, 0), (7, 0), (4099, 0), ((1 << 20) + 3, 0), (1031, 1)]


def same(a, b):
    """Bit equality, with any NaN equal to any NaN (the device's canonical
    NaN and glibc's differ in sign)."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def inputs(fn, n, seed):
    g = SplitMix64(seed)
    if fn in (FN_SQRT, FN_RSQRT, FN_LOG):
        x = np.exp(g.uniform((n,), -60.0, 60.0)).astype(np.float32)
    elif fn == FN_EXP:
        x = g.uniform((n,), -87.0, 88.0)
    elif fn in (FN_SIN, FN_COS):
        x = g.uniform((n,), -200.0, 200.0)
        x[: n // 2] = g.uniform((n // 2,), -1e5, 1e5)  # large arguments need a full range reduction
    elif fn == FN_ERF:
        x = g.uniform((n,), -5.0, 5.0)
    else:
        x = g.normal((n,), 0.0, 100.0)
    return np.ascontiguousarray(x, np.float32)


def run(fn, x, off=0):
    dx, dz = dev(x, off), empty(x.shape, offset_floats=off)
    call("cxm_wise_f32", dx.ptr, dz.ptr, x.size, fn, None)
    return dz.numpy()


EXACT = [FN_SQUARE, FN_ABS, FN_NEG, FN_SIGN, FN_SQRT, FN_RCP, FN_INVERSE]
F64 = {FN_RSQRT: lambda d: 1.0 / np.sqrt(d), FN_LOG: np.log, FN_EXP: np.exp, FN_ERF: scipy.special.erf,
       FN_SIN: np.sin, FN_COS: np.cos}


@pytest.mark.parametrize("fn", EXACT)
@pytest.mark.parametrize("n,off", SIZES)
def test_exact_functions(hip, orc, fn, n, off):
    x = inputs(fn, n, 100 + fn * 7 + n)
    assert same(run(fn, x, off), orc.wise(x, fn))


@pytest.mark.parametrize("fn", sorted(F64))
@pytest.mark.parametrize("n,off", SIZES)
def test_transcendentals_within_2ulp(hip, orc, fn, n, off):
    x = inputs(fn, n, 200 + fn * 7 + n)
    got = run(fn, x, off)
    exact = F64[fn](x.astype(np.float64)).astype(np.float32)
    d = ulp_dist(got, exact)
    assert d.max() <= 2, (fn, x[d.argmax()], got[d.argmax()], exact[d.argmax()])
    assert ulp_dist(got, orc.wise(x, fn)).max() <= 3  # the oracle is itself within 1 ulp


def test_special_values(hip, orc):
    x = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, -1.0, 1.0, 2.0, 1e-40], np.float32)
    r = {fn: run(fn, x) for fn in range(13)}
    assert same(r[FN_SQRT][:7], [0.0, -0.0, np.inf, np.nan, np.nan, np.nan, 1.0])
    assert same(r[FN_RSQRT][:7], [np.inf, -np.inf, 0.0, np.nan, np.nan, np.nan, 1.0])
    assert same(r[FN_LOG][:7], [-np.inf, -np.inf, np.inf, np.nan, np.nan, np.nan, 0.0])
    assert same(r[FN_EXP][:5], [1.0, 1.0, np.inf, 0.0, np.nan])
    assert same(r[FN_ERF][:5], [0.0, -0.0, 1.0, -1.0, np.nan])
    assert same(r[FN_SIN][:5], [0.0, -0.0, np.nan, np.nan, np.nan])
    assert same(r[FN_COS][:5], [1.0, 1.0, np.nan, np.nan, np.nan])
    assert same(r[FN_RCP][:4], [np.inf, -np.inf, 0.0, -0.0])
    assert same(r[FN_SIGN], [0.0, 0.0, 1.0, -1.0, 0.0, -1.0, 1.0, 1.0, 1.0])
    assert same(r[FN_ABS][:4], [0.0, 0.0, np.inf, np.inf]) and not np.signbit(r[FN_ABS][1])
    for fn in EXACT:  # the exact functions agree with the oracle on every special value
        assert same(r[fn], orc.wise(x, fn)), fn


def test_in_place(hip, orc):
    x = inputs(FN_LOG, 100003, 5)
    d = dev(x)
    engine.wise.log(d, d)
    assert ulp_dist(d.numpy(), np.log(x.astype(np.float64)).astype(np.float32)).max() <= 2
    before = d.numpy()
    engine.wise.neg(d, d)
    assert same(d.numpy(), -before)
    engine.wise.abs(d, d)
    assert same(d.numpy(), np.abs(before))


@pytest.mark.parametrize("n,off", [(5, 0), (100003, 0), (1031, 1)])
def test_pow_tensor_and_scalar(hip, orc, n, off):
    g = SplitMix64(300 + n)
    x = g.uniform((n,), 0.01, 10.0)
    y = g.uniform((n,), -6.0, 6.0)
    dx, dy, dz = dev(x, off), dev(y, off), empty((n,), offset_floats=off)
    call("cxm_binary_f32", dx.ptr, dy.ptr, dz.ptr, n, OP_POW, None)
    exact = np.power(x.astype(np.float64), y.astype(np.float64)).astype(np.float32)
    assert ulp_dist(dz.numpy(), exact).max() <= 2
    call("cxm_scalar_f32", dx.ptr, np.float32(2.5), dz.ptr, n, OP_POW, None)
    exact = np.power(x.astype(np.float64), 2.5).astype(np.float32)
    assert ulp_dist(dz.numpy(), exact).max() <= 2


def test_pow_special_values(hip, orc):
    x = np.array([-2.0, -2.0, 0.0, 1.0, 5.0, np.nan, 2.0, -0.0], np.float32)
    y = np.array([3.0, 0.5, -1.0, np.nan, 0.0, 0.0, 10.0, 3.0], np.float32)
    dx, dy, dz = dev(x), dev(y), empty((8,))
    call("cxm_binary_f32", dx.ptr, dy.ptr, dz.ptr, 8, OP_POW, None)
    z = dz.numpy()
    assert same(z, [-8.0, np.nan, np.inf, 1.0, 1.0, 1.0, 1024.0, -0.0])
    assert same(z, orc.binary(x, y, OP_POW))


@pytest.mark.parametrize("n,off", [(3, 0), (100003, 0), (1031, 1)])
def test_lerp_clamp(hip, orc, n, off):
    x = SplitMix64(400 + n).normal((n,), 0.0, 10.0)
    x[:3] = [np.nan, np.inf, -np.inf][: min(3, n)]
    dx, dz = dev(x, off), empty((n,), offset_floats=off)
    call("cxm_lerp_f32", dx.ptr, np.float32(3.3), np.float32(0.7), dz.ptr, n, None)
    assert same(dz.numpy(), orc.lerp(x, 3.3, 0.7))
    call("cxm_clamp_f32", dx.ptr, np.float32(-1.5), np.float32(2.0), dz.ptr, n, None)
    assert same(dz.numpy(), orc.clamp(x, -1.5, 2.0))


@pytest.mark.parametrize("dtype", [np.float32, np.int32])
@pytest.mark.parametrize("xn,n", [(1, 1), (1000, 5000), (1 << 20, 1 << 20)])
def test_gather(hip, orc, dtype, xn, n):
    g = SplitMix64(500 + n)
    if dtype == np.float32:
        x = g.normal((xn,))
    else:
        x = (g.uniform((xn,), -1e6, 1e6)).astype(np.int32)
    idx = (g.uniform((n,), 0.0, 1.0) * xn).astype(np.int64).clip(0, xn - 1).astype(np.int32)
    idx[: min(n, 2)] = [-1, xn][: min(n, 2)]  # out of range: NaN / INT32_MIN, no read
    d_x, d_i, d_z = dev(x), dev(idx), empty((n,), dtype)
    engine.wise.gather(d_x, d_i, d_z, n)
    got, ref = d_z.numpy(), orc.gather(x, idx)
    if dtype == np.float32:
        assert same(got, ref)
    else:
        assert np.array_equal(got, ref)


def test_argument_errors(hip):
    d = empty((4,))
    assert lib().cxm_wise_f32(d.ptr, d.ptr, 4, 13, None) == E_INVALID
    assert lib().cxm_wise_f32(d.ptr, d.ptr, 4, -1, None) == E_INVALID
    assert lib().cxm_wise_f32(None, d.ptr, 4, 0, None) == E_INVALID
    assert lib().cxm_bcast_row_f32(d.ptr, d.ptr, d.ptr, 2, 2, OP_POW, None) == E_INVALID
    assert lib().cxm_gather_f32(d.ptr, 4, None, d.ptr, 4, None) == E_INVALID
    assert lib().cxm_wise_f32(d.ptr, d.ptr, 0, 0, None) == 0


def test_pow_wide_range(hip):
    """pow over the ranges where its logarithm must be carried in double-float:
    |x| at the edges of the reduction interval (about 0.707 and 1.414) with
    |y| up to 140, x from 1e-38 to 1e38, x near 1 with |y| up to 1000, and
    subnormal results; finite results within 2 ulp of float64 (subnormal
    ones in units of the subnormal spacing)."""
    g = SplitMix64(0x90)
    xs = [g.uniform((1 << 16,), 0.69, 0.72), g.uniform((1 << 16,), 1.40, 1.43),
          (10.0 ** g.uniform((1 << 16,), -38.0, 38.0)).astype(np.float32), g.uniform((1 << 16,), 0.9, 1.1),
          g.uniform((1 << 16,), 0.5, 2.0)]
    ys = [g.uniform((1 << 16,), -140.0, 140.0), g.uniform((1 << 16,), -140.0, 140.0),
          g.uniform((1 << 16,), -1.5, 1.5), g.uniform((1 << 16,), -1000.0, 1000.0),
          g.uniform((1 << 16,), -200.0, -120.0)]
    x = np.concatenate(xs).astype(np.float32)
    y = np.concatenate(ys).astype(np.float32)
    dx, dy, dz = dev(x), dev(y), empty(x.shape)
    call("cxm_binary_f32", dx.ptr, dy.ptr, dz.ptr, x.size, OP_POW, None)
    got = dz.numpy()
    with np.errstate(over="ignore", under="ignore"):
        ref64 = np.power(x.astype(np.float64), y.astype(np.float64))
    ref = ref64.astype(np.float32)
    fin = np.isfinite(ref) & (np.abs(ref64) < 3.4e38)
    spacing = np.maximum(np.spacing(np.abs(ref[fin])).astype(np.float64), 2.0 ** -149)
    err = np.abs(got[fin].astype(np.float64) - ref64[fin]) / spacing
    assert err.max() <= 2.0, float(err.max())
    big = ~fin & (ref64 > 0)
    assert np.all(np.isinf(got[big])), "overflowing results must be +inf"


def test_pow_special_value_table(hip):
    """The IEEE / C99 special cases of pow, against numpy's float32 power
    (the C library's powf): every pair from a set of zeros, ones,
    infinities, NaN, integers (odd, even), non-integers and subnormals of
    both signs."""
    vals = np.array([0.0, -0.0, 1.0, -1.0, 2.0, -2.0, 0.5, -0.5, 3.0, -3.0, 2.5, -2.5, np.inf, -np.inf, np.nan,
                     1e-40, -1e-40, 1e30, -1e30, 7.0, 2.0 ** 24, 2.0 ** 25 + 2.0], np.float32)
    x = np.repeat(vals, vals.size)
    y = np.tile(vals, vals.size)
    dx, dy, dz = dev(x), dev(y), empty(x.shape)
    call("cxm_binary_f32", dx.ptr, dy.ptr, dz.ptr, x.size, OP_POW, None)
    got = dz.numpy()
    with np.errstate(all="ignore"):
        want = np.power(x, y)  # float32 powf
    bad = []
    for i in range(x.size):
        a, b = got[i], want[i]
        if np.isnan(b):
            ok = np.isnan(a)
        elif np.isinf(b) or b == 0:
            ok = a == b and np.signbit(a) == np.signbit(b)
        else:
            ok = abs(float(a) - float(b)) <= 2 * float(np.spacing(np.abs(b)))
        if not ok:
            bad.append((float(x[i]), float(y[i]), float(a), float(b)))
    assert not bad, bad[:10]
