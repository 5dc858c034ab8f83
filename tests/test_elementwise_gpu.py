"""Parity of the gfx950 elementwise, broadcast, activation, affine and SGD
kernels with the CPU oracle.

Bars: add/sub/mul/div/max/min, ReLU and every broadcast are bit-exact
(single IEEE rounding per operation, no fma); sigmoid and tanh are within
2 ulp of the float64 function of the same fp32 pre-activation; column sums
(dscale, dbias) within 1e-5 * sum of |terms|.
"""
import numpy as np
import pytest

from cortexmind_amd import engine
from cortexmind_amd._lib import (ACT_EXP, ACT_NONE, ACT_RELU, ACT_SIGMOID, ACT_TANH, OP_ADD,
                                 OP_DIV, OP_MAX, OP_MIN, OP_MUL, OP_SUB, call)
from cortexmind_amd.data import SplitMix64, c3_affine

from gpu_util import bits_equal, dev, empty, ulp_dist

pytestmark = pytest.mark.gpu

OPS = [OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_MAX, OP_MIN]


def special_values(n, seed):
    x = SplitMix64(seed).normal((n,), 0.0, 3.0)
    sp = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 88.0, -88.0, 1e30], np.float32)
    x[: min(n, sp.size)] = sp[: min(n, sp.size)]
    return x


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("n,off", [(1, 0), (5, 0), (4099, 0), (1000003, 0), (1031, 1)])
def test_binary(hip, orc, op, n, off):
    x = special_values(n, 11 + n)
    y = SplitMix64(12 + n).normal((n,), 0.0, 2.0)
    dx, dy, dz = dev(x, off), dev(y, off), empty((n,), offset_floats=off)
    call("cxm_binary_f32", dx.ptr, dy.ptr, dz.ptr, n, op, None)
    assert bits_equal(dz.numpy(), orc.binary(x, y, op))


def test_binary_in_place(hip, orc):
    x = SplitMix64(3).normal((4096,))
    y = SplitMix64(4).normal((4096,))
    dx, dy = dev(x), dev(y)
    engine.matrix_t.mul(dx, dy, 4096)  # the in-place form writes Xx
    assert bits_equal(dx.numpy(), orc.binary(x, y, OP_MUL))


@pytest.mark.parametrize("op", [OP_ADD, OP_SUB, OP_MUL, OP_DIV])
@pytest.mark.parametrize("mode", ["row", "col"])
@pytest.mark.parametrize("m,n,off", [(512, 1024, 0), (37, 64, 0), (6, 280, 0), (13, 1028, 0), (5, 37, 0), (3, 8, 1),
                                     (1, 1, 0)])
def test_broadcast(hip, orc, op, mode, m, n, off):
    x = SplitMix64(m * 7 + n).normal((m, n), 0.0, 2.0)
    y = SplitMix64(m + n * 3).uniform((n if mode == "row" else m,), 0.5, 1.5)
    dx, dy, dz = dev(x, off), dev(y), empty((m, n), offset_floats=off)
    call(f"cxm_bcast_{mode}_f32", dx.ptr, dy.ptr, dz.ptr, m, n, op, None)
    ref = orc.bcast_row(x, y, op) if mode == "row" else orc.bcast_col(x, y, op)
    assert bits_equal(dz.numpy(), ref)


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("n,off", [(7, 0), (100003, 0), (257, 1)])
def test_scalar(hip, orc, op, n, off):
    x = special_values(n, 21 + n)
    dx, dz = dev(x, off), empty((n,), offset_floats=off)
    call("cxm_scalar_f32", dx.ptr, np.float32(0.37), dz.ptr, n, op, None)
    assert bits_equal(dz.numpy(), orc.scalar(x, np.float32(0.37), op))


@pytest.mark.parametrize("n,off", [(10, 0), (1 << 20, 0), (1001, 1)])
def test_relu_exact(hip, orc, n, off):
    x = special_values(n, 31 + n)
    dx, dz = dev(x, off), empty((n,), offset_floats=off)
    call("cxm_unary_f32", dx.ptr, dz.ptr, n, ACT_RELU, None)
    got = dz.numpy()
    assert bits_equal(got, orc.unary(x, ACT_RELU))
    if n >= 2:  # relu(-0.0) = -0.0 and relu(NaN) = NaN, as _mm256_max_ps(0, x)
        assert np.signbit(got[1]) and got[1] == 0.0
    if n >= 5:
        assert np.isnan(got[4])


def f64_act(t, act):
    t = t.astype(np.float64)
    with np.errstate(over="ignore"):
        if act == ACT_SIGMOID:
            return (1.0 / (1.0 + np.exp(-t))).astype(np.float32)
        if act == ACT_TANH:
            return np.tanh(t).astype(np.float32)
        return np.exp(t).astype(np.float32)


@pytest.mark.parametrize("act", [ACT_SIGMOID, ACT_TANH, ACT_EXP])
def test_transcendental_ulp(hip, act):
    g = SplitMix64(41 + act)
    # sigmoid's results reach the denormal range below t = -87.3 and 0 below
    # about -103.3; 1 + e^-t overflows below -88.7
    x = np.concatenate([g.normal((1 << 20,), 0.0, 4.0), g.uniform((1 << 18,), -87.0, 88.0),
                        g.uniform((1 << 16,), -110.0, -80.0),
                        np.array([0.0, -0.0, 1e-30, -1e-30, 20.0, -20.0, 9.0, -9.0, -88.7, -88.8, -100.0,
                                  -150.0, np.inf, -np.inf], np.float32)])
    dx, dz = dev(x), empty(x.shape)
    call("cxm_unary_f32", dx.ptr, dz.ptr, x.size, act, None)
    got = dz.numpy()
    ref = f64_act(x, act)
    fin = np.isfinite(ref)
    assert np.all(ulp_dist(got[fin], ref[fin]) <= 2), int(ulp_dist(got[fin], ref[fin]).max())


# ----------------------------------------------------------- C3 affine

@pytest.fixture(scope="module")
def c3_small():
    g = SplitMix64(0xC3)
    m, n = 300, 1028
    return (g.normal((m, n)), g.uniform((n,), 0.5, 1.5), g.normal((n,), 0.0, 0.1), g.normal((m, n)))


def affine_fwd_gpu(x, s, b, act, off=0):
    m, n = x.shape
    dx, ds, db, dy = dev(x, off), dev(s), dev(b), empty((m, n), offset_floats=off)
    engine.activation.affine_fwd(dx, ds, db, dy, m, n, act)
    return dy.numpy()


def affine_bwd_gpu(x, s, y, g, act):
    m, n = x.shape
    dx_, ds_, dy_, dg_ = dev(x), dev(s), dev(y), dev(g)
    ddx, dds, ddb = empty((m, n)), empty((n,)), empty((n,))
    engine.activation.affine_bwd(dx_, ds_, dy_, dg_, ddx, dds, ddb, m, n, act)
    return ddx.numpy(), dds.numpy(), ddb.numpy()


def check_fwd(x, s, b, act, y, orc):
    if act in (ACT_RELU, ACT_NONE):
        assert bits_equal(y, orc.affine_act_fwd(x, s, b, act))
    else:
        t = (x * s[None, :]).astype(np.float32) + b[None, :]
        t = t.astype(np.float32)
        ref = f64_act(t, act)
        assert int(ulp_dist(y, ref).max()) <= 2


def check_bwd(x, s, y, g, act, got, orc):
    dx, ds, db = got
    rdx, rds, rdb = orc.affine_act_bwd(x, s, y, g, act)
    assert bits_equal(dx, rdx)
    # bound from the terms' magnitudes (|dz| <= |dy| since |act'| <= 1)
    dz_abs = np.abs(g.astype(np.float64))
    assert np.all(np.abs(ds.astype(np.float64) - rds) <= 1e-5 * (np.abs(x) * dz_abs).sum(axis=0) + 1e-30)
    assert np.all(np.abs(db.astype(np.float64) - rdb) <= 1e-5 * dz_abs.sum(axis=0) + 1e-30)


@pytest.mark.parametrize("act", [ACT_NONE, ACT_RELU, ACT_SIGMOID, ACT_TANH])
@pytest.mark.parametrize("off", [0, 1])
def test_affine_small(hip, orc, c3_small, act, off):
    x, s, b, g = c3_small
    if off:
        x, s, b, g = x[:, :-3].copy(), s[:-3].copy(), b[:-3].copy(), g[:, :-3].copy()  # n = 1025, scalar path
    y = affine_fwd_gpu(x, s, b, act, off)
    check_fwd(x, s, b, act, y, orc)
    check_bwd(x, s, y, g, act, affine_bwd_gpu(x, s, y, g, act), orc)


@pytest.mark.parametrize("act", [ACT_RELU, ACT_SIGMOID, ACT_TANH])
@pytest.mark.parametrize("m,n", [(7, 264), (1, 4), (5, 2056)])
def test_affine_ragged(hip, orc, act, m, n):
    """Row counts off a multiple of four and rows of 66, 1 and 514 float4
    (a partial last 64-float4 column tile) on the vector path."""
    g = SplitMix64(0xA5 + m + n)
    x, s, b, dy = g.normal((m, n)), g.uniform((n,), 0.5, 1.5), g.normal((n,), 0.0, 0.1), g.normal((m, n))
    y = affine_fwd_gpu(x, s, b, act)
    check_fwd(x, s, b, act, y, orc)
    check_bwd(x, s, y, dy, act, affine_bwd_gpu(x, s, y, dy, act), orc)


@pytest.mark.parametrize("act", [ACT_RELU, ACT_SIGMOID, ACT_TANH])
def test_affine_c3_full(hip, orc, act):
    """C3 at its full size [8192, 8192]."""
    x, s, b, g = c3_affine()
    y = affine_fwd_gpu(x, s, b, act)
    check_fwd(x, s, b, act, y, orc)
    check_bwd(x, s, y, g, act, affine_bwd_gpu(x, s, y, g, act), orc)


@pytest.mark.parametrize("n,off", [(10, 0), (784 * 1024, 0), (1025, 1)])
def test_sgd(hip, orc, n, off):
    w = SplitMix64(51 + n).normal((n,))
    gr = SplitMix64(52 + n).normal((n,))
    dw, dg = dev(w, off), dev(gr, off)
    call("cxm_sgd_f32", dw.ptr, dg.ptr, np.float32(0.01), n, None)
    assert bits_equal(dw.numpy(), orc.sgd(w, gr, 0.01))


@pytest.mark.parametrize("act", [ACT_RELU, ACT_SIGMOID, ACT_TANH])
@pytest.mark.parametrize("n,off", [(1, 0), (4099, 0), (1 << 20, 0), (1031, 1)])
def test_act_bwd_bit_exact(hip, orc, act, n, off):
    """dx = dy * act'(y) from the saved output (what a ReLU/sigmoid/tanh
    GradientFlow runs): one rounded factor, one product, bit-exact."""
    x = SplitMix64(700 + n + act).normal((n,), 0.0, 2.0)
    y = orc.unary(x, act)
    y[: min(n, 3)] = np.array([0.0, -0.0, 1.0], np.float32)[: min(n, 3)]  # relu' at 0 and -0 is 0
    dy = SplitMix64(800 + n).normal((n,), 0.0, 1.0)
    d_y, d_dy, d_dx = dev(y, off), dev(dy, off), empty((n,), offset_floats=off)
    call("cxm_act_bwd_f32", d_y.ptr, d_dy.ptr, d_dx.ptr, n, act, None)
    assert bits_equal(d_dx.numpy(), orc.act_bwd(y, dy, act))


def test_tanh_ranges(hip):
    """tanh (the library's two-range form): dense around the polynomial /
    exponential switch at |t| = 0.9 (every float within 4096 ulps of it),
    uniform on [-1.5, 1.5], tiny and denormal arguments (tanh(t) = t), and
    the special values: +-0 keep their sign, +-inf give +-1, NaN stays NaN."""
    g = SplitMix64(0x7A2)
    sweep = np.float32(0.9).view(np.int32) + np.arange(-4096, 4097, dtype=np.int32)
    near = sweep.view(np.float32)
    x = np.concatenate([near, -near, g.uniform((1 << 20,), -1.5, 1.5), g.uniform((1 << 16,), 1e-8, 1e-3),
                        np.array([1e-38, -1e-38, 1e-45, -1e-45, 3e-41], np.float32)]).astype(np.float32)
    dx, dz = dev(x), empty(x.shape)
    call("cxm_unary_f32", dx.ptr, dz.ptr, x.size, ACT_TANH, None)
    got = dz.numpy()
    ref = f64_act(x, ACT_TANH)
    assert np.all(ulp_dist(got, ref) <= 2), int(ulp_dist(got, ref).max())
    sp = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 9.5, -9.5, 1e30, -1e30], np.float32)
    dx, dz = dev(sp), empty(sp.shape)
    call("cxm_unary_f32", dx.ptr, dz.ptr, sp.size, ACT_TANH, None)
    got = dz.numpy()
    assert got[0] == 0.0 and not np.signbit(got[0]) and got[1] == 0.0 and np.signbit(got[1])
    assert got[2] == 1.0 and got[3] == -1.0 and np.isnan(got[4])
    assert list(got[5:]) == [1.0, -1.0, 1.0, -1.0]
