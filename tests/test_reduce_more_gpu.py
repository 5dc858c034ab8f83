"""Parity of the gfx950 min / argmin / norm1 / norm2 / var / stdv reductions
(reference: avx2::reduce, source/CortexMind/framework/Engine/AVX2/
reduce.cpp:86-437, 530-621) with the CPU oracle and float64.

Bars: min and argmin bit-exact (first index on ties).  norm1, norm2, var
and stdv sum positive terms, so the bar is relative to the result itself:
within 1e-5 of the float64 value at every size, and within 1e-5 of the
oracle at sizes where the oracle's own sequential fp32 accumulation is that
accurate (up to 2^16 terms per output; at 2^24 terms its lanes drift by
~1e-4, which is the reference's error, not the device's).
"""
import numpy as np
import pytest

from cortexmind_amd import engine
from cortexmind_amd._lib import E_INVALID, call, lib
from cortexmind_amd.data import SplitMix64, c2_reduce
from cortexmind_amd.device import DeviceArray

pytestmark = pytest.mark.gpu

REL = 1e-5
ORACLE_MAX_TERMS = 1 << 16


def gpu_reduce(op, x, sizes, ptr_offset_floats=0):
    flat = np.ascontiguousarray(x, np.float32).ravel()
    buf = np.concatenate([np.zeros(ptr_offset_floats, np.float32), flat])
    dx = DeviceArray.from_numpy(buf)
    n_out = 1 if len(sizes) == 1 else sizes[0] * sizes[2]
    dz = DeviceArray((n_out,), np.int32 if op == "argmin" else np.float32)
    xp = dx.ptr + 4 * ptr_offset_floats
    if len(sizes) == 1:
        call(f"cxm_reduce_{op}_flat_f32", xp, dz.ptr, sizes[0], None)
    else:
        call(f"cxm_reduce_{op}_f32", xp, dz.ptr, *sizes, None)
    return dz.numpy()


def exact(op, x, sizes):
    d = np.asarray(x, np.float64)
    d = d.reshape(1, -1, 1) if len(sizes) == 1 else d.reshape(sizes)
    if op == "norm1":
        r = np.abs(d).sum(axis=1)
    elif op == "norm2":
        r = np.sqrt((d * d).sum(axis=1))
    elif op == "var":
        r = d.var(axis=1)
    else:
        r = d.std(axis=1)
    return r.ravel()


def check(op, x, sizes, orc, vs_oracle=True, **kw):
    got = gpu_reduce(op, x, sizes, **kw)
    ref = orc.reduce_flat(op, x) if len(sizes) == 1 else None
    dim = sizes[0] if len(sizes) == 1 else sizes[1]
    if op in ("min", "argmin"):
        ref = orc.reduce_flat(op, x) if len(sizes) == 1 else orc.reduce_axis(op, x, *sizes)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (op, sizes)
        return got
    e = exact(op, x, sizes)
    err = np.abs(got.astype(np.float64) - e)
    assert np.all(err <= REL * np.abs(e) + 1e-37), (op, sizes, float(np.max(err / np.maximum(np.abs(e), 1e-30))))
    if vs_oracle and dim <= ORACLE_MAX_TERMS:
        ref = orc.reduce_flat(op, x) if len(sizes) == 1 else orc.reduce_axis(op, x, *sizes)
        assert np.all(np.abs(got.astype(np.float64) - ref) <= REL * np.abs(e) + 1e-37), (op, sizes)
    return got


OPS = ["min", "argmin", "norm1", "norm2", "var", "stdv"]


@pytest.fixture(scope="module")
def c2():
    return c2_reduce()


@pytest.mark.parametrize("op", OPS)
def test_c2_global(hip, orc, c2, op):
    check(op, c2, (c2.size,), orc)


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("axis", [0, 1])
def test_c2_axis(hip, orc, c2, op, axis):
    check(op, c2, (1, 4096, 4096) if axis == 0 else (4096, 4096, 1), orc)


@pytest.mark.parametrize("n", [1, 3, 8, 9, 1023, 4099, 65537, (1 << 20) + 3])
@pytest.mark.parametrize("op", OPS)
def test_flat_ragged(hip, orc, n, op):
    check(op, SplitMix64(50 + n).normal((n,), 1.5, 3.0), (n,), orc)


@pytest.mark.parametrize("op", OPS)
def test_flat_unaligned_pointer(hip, orc, op):
    check(op, SplitMix64(78).uniform((10001,), -1, 1), (10001,), orc, ptr_offset_floats=1)


@pytest.mark.parametrize("sizes", [(7, 9, 1), (3, 1025, 1), (64, 131072, 1), (1, 7, 3), (2, 5, 9),
                                   (1, 257, 33), (3, 64, 17), (2, 100, 1000), (4, 4, 4096),
                                   (1, 3000, 260), (1, 3, 9)])
@pytest.mark.parametrize("op", OPS)
def test_axis_shapes(hip, orc, sizes, op):
    o, d, i = sizes
    check(op, SplitMix64(o * 7919 + d * 31 + i).normal((o, d, i), -0.5, 2.0), sizes, orc)


def test_var_large_mean_small_spread(hip, orc):
    # mean 1000, spread 0.01: a one-pass fp32 sum-of-squares formula loses
    # every digit here.  The second case makes the first element (the shift)
    # an outlier 1000 spreads away from the mean.  Bar: the exact value
    # only.  The reference's own fp32 mean (8 lanes of 512-term sums near
    # 5e5, reduce.cpp:112-120) is off by a sizeable part of the spread, so
    # its variance is not a usable target on such data.
    x = (1000.0 + SplitMix64(9).normal((1 << 20,), 0.0, 0.01)).astype(np.float32)
    for sizes in [(x.size,), (256, 4096, 1), (1, 4096, 256)]:
        check("var", x, sizes, orc, vs_oracle=False)
    y = x.copy()
    y[:256] = 1010.0  # row 0 of the column layout and element 0 of every layout
    for sizes in [(y.size,), (1, 4096, 256)]:
        check("var", y, sizes, orc, vs_oracle=False)


def test_var_column_scaling_kat(hip):
    # columns (0.5, 2.5, 3.0): m2 = 3.5 exactly; the first 8 of 9 column
    # outputs multiply by rn(1/3) (0x3f955556), the 9th divides (0x3f955555);
    # rows divide (reduce.cpp:135, 173-182)
    x = np.repeat(np.array([0.5, 2.5, 3.0], np.float32), 9).reshape(3, 9)
    z = gpu_reduce("var", x, (1, 3, 9))
    assert [hex(v) for v in z.view(np.uint32)] == ["0x3f955556"] * 8 + ["0x3f955555"]
    r = gpu_reduce("var", np.tile(np.array([0.5, 2.5, 3.0], np.float32), 4), (4, 3, 1))
    assert [hex(v) for v in r.view(np.uint32)] == ["0x3f955555"] * 4


def test_min_argmin_semantics(hip, orc):
    x = np.zeros((6, 40), np.float32)
    x[1, [3, 17, 39]] = -5.0         # repeated minimum -> first one
    x[2, :] = 1.0                    # all equal -> 0
    x[3, [0, 39]] = -2.0
    x[4, 10:] = -7.0
    x[5, :] = np.inf                 # all +inf
    for sizes in [(6, 40, 1), (1, 6, 40)]:
        check("argmin", x, sizes, orc)
        check("min", x, sizes, orc)
    check("argmin", x.ravel(), (x.size,), orc)
    row = gpu_reduce("min", x, (6, 40, 1))
    assert row[5] == np.finfo(np.float32).max  # flat/row forms start from FLT_MAX
    col = gpu_reduce("min", np.full((4, 16), np.inf, np.float32), (1, 4, 16))
    assert np.all(np.isposinf(col))            # column form starts from slice 0


def test_flat_zero_elements(hip):
    z = DeviceArray((1,), np.float32)
    for op, want in [("norm1", 0.0), ("norm2", 0.0), ("min", np.finfo(np.float32).max)]:
        call(f"cxm_reduce_{op}_flat_f32", None, z.ptr, 0, None)
        assert z.numpy()[0] == np.float32(want)
    for op in ("var", "stdv"):
        call(f"cxm_reduce_{op}_flat_f32", None, z.ptr, 0, None)
        assert np.isnan(z.numpy()[0])
    assert lib().cxm_reduce_argmin_flat_f32(None, z.ptr, 0, None) == E_INVALID


def test_engine_mirror_names(hip, orc):
    x = SplitMix64(6).uniform((3, 50, 8), -1, 1)
    dx = DeviceArray.from_numpy(x)
    dz = DeviceArray((24,), np.float32)
    engine.reduce.min(dx, dz, 3, 50, 8)
    assert np.array_equal(dz.numpy(), orc.reduce_axis("min", x, 3, 50, 8))
    di = DeviceArray((24,), np.int32)
    engine.reduce.argmin(dx, di, 3, 50, 8)
    assert np.array_equal(di.numpy(), orc.reduce_axis("argmin", x, 3, 50, 8))
    engine.reduce.var(dx, dz, x.size)
    assert abs(dz.numpy()[0] - x.astype(np.float64).var()) <= REL * x.astype(np.float64).var()
