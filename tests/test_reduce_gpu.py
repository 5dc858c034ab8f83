"""Parity of the gfx950 reductions with the CPU oracle (a restatement of
avx2::reduce, source/CortexMind/framework/Engine/AVX2/reduce.cpp).

Bars (from the task's parity contract): max and argmax bit-exact; sum and
mean within |gpu - ref| <= 1e-5 * sum|x| per output, because the GPU adds
in a tree and the reference in 8 sequential lanes (both round, differently).
"""
import ctypes

import numpy as np
import pytest

from cortexmind_amd import engine
from cortexmind_amd._lib import E_INVALID, call, lib
from cortexmind_amd.data import SplitMix64, c2_reduce
from cortexmind_amd.device import DeviceArray

pytestmark = pytest.mark.gpu

SUM_TOL = 1e-5


def gpu_reduce(op, x, sizes, ptr_offset_floats=0):
    """Run one reduction on the device; sizes = (n,) or (outer, dim, inner)."""
    flat = np.ascontiguousarray(x, np.float32).ravel()
    buf = np.concatenate([np.zeros(ptr_offset_floats, np.float32), flat])
    dx = DeviceArray.from_numpy(buf)
    n_out = 1 if len(sizes) == 1 else sizes[0] * sizes[2]
    dz = DeviceArray((n_out,), np.int32 if op in ("argmax", "argmin") else np.float32)
    xp = dx.ptr + 4 * ptr_offset_floats
    if len(sizes) == 1:
        call(f"cxm_reduce_{op}_flat_f32", xp, dz.ptr, sizes[0], None)
    else:
        call(f"cxm_reduce_{op}_f32", xp, dz.ptr, *sizes, None)
    return dz.numpy()


def abs_sums(x, sizes):
    a = np.abs(np.asarray(x, np.float64)).ravel()
    if len(sizes) == 1:
        return np.array([a.sum()])
    o, d, i = sizes
    return a.reshape(o, d, i).sum(axis=1).ravel()


def check(op, x, sizes, orc, **kw):
    got = gpu_reduce(op, x, sizes, **kw)
    ref = orc.reduce_flat(op, x) if len(sizes) == 1 else orc.reduce_axis(op, x, *sizes)
    if op in ("max", "argmax", "min", "argmin"):
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (op, sizes)
    else:
        tol = SUM_TOL * abs_sums(x, sizes)
        if op == "mean":
            tol = tol / sizes[1 if len(sizes) == 3 else 0]
        err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
        assert np.all(err <= tol + 1e-30), (op, sizes, float(np.max(err - tol)))
    return got, ref


# ------------------------------------------------------------- C2 full size

@pytest.fixture(scope="module")
def c2():
    return c2_reduce()


@pytest.mark.parametrize("op", ["sum", "mean", "max", "argmax"])
def test_c2_global(hip, orc, c2, op):
    if op in ("max", "argmax"):
        check(op, c2, (c2.size,), orc)
    else:
        got, _ = check(op, c2, (c2.size,), orc)
        exact = np.sum(c2.astype(np.float64))
        if op == "mean":
            exact /= c2.size
        # the GPU's own error against float64 is well inside the bar too
        assert abs(got[0] - exact) <= SUM_TOL * np.abs(c2.astype(np.float64)).sum() / (
            c2.size if op == "mean" else 1)


@pytest.mark.parametrize("op", ["sum", "mean", "max", "argmax"])
@pytest.mark.parametrize("axis", [0, 1])
def test_c2_axis(hip, orc, c2, op, axis):
    sizes = (1, 4096, 4096) if axis == 0 else (4096, 4096, 1)
    check(op, c2, sizes, orc)


@pytest.mark.parametrize("n", [4096 * 4096, 4096 * 4096 + 3, 1 << 22])
def test_global_sum_exact_integers(hip, n):
    """Full-size global sum and mean of integers in {-1, 0, 1}: every partial
    sum is an integer below 2^24 in magnitude, so each is exact in fp32 and
    the result must equal the exact sum bit for bit.  A lost or doubled
    segment partial (std ~52 for 8192 such terms) cannot hide under this bar,
    where it could under the 1e-5 * sum|x| tolerance of U(-1, 1) data.
    Flat and (1, n, 1) forms; the odd length also runs the scalar tail."""
    r = SplitMix64(0xE1 + n).next_u64(n)
    x = ((r % np.uint64(3)).astype(np.int64) - 1).astype(np.float32)
    exact = int(np.sum(x.astype(np.int64)))
    assert abs(exact) < (1 << 24)
    for sizes in [(n,), (1, n, 1)]:
        got = gpu_reduce("sum", x, sizes)
        assert got[0] == np.float32(exact), (sizes, float(got[0]), exact)
        mean = gpu_reduce("mean", x, sizes)
        # flat: sum / (float)N; axis with one output: the division tail
        want = np.float32(exact) / np.float32(n)
        assert mean[0] == want, (sizes, float(mean[0]), float(want))


@pytest.mark.parametrize("sizes", [(4096, 4096, 1), (1, 4096, 4096), (3, 1000, 257)])
def test_axis_sum_exact_integers(hip, sizes):
    """Row and column sums of integers in {-1, 0, 1}: exact, bit for bit."""
    o, d, i = sizes
    r = SplitMix64(0xE2 + d).next_u64(o * d * i)
    x = ((r % np.uint64(3)).astype(np.int64) - 1).astype(np.float32).reshape(o, d, i)
    exact = x.astype(np.int64).sum(axis=1).ravel().astype(np.float32)
    got = gpu_reduce("sum", x, sizes)
    assert np.array_equal(got, exact), sizes


def test_c2_deterministic(hip, c2):
    a = gpu_reduce("sum", c2, (c2.size,))
    b = gpu_reduce("sum", c2, (c2.size,))
    c = gpu_reduce("sum", c2, (1, 4096, 4096))
    d = gpu_reduce("sum", c2, (1, 4096, 4096))
    assert a.tobytes() == b.tobytes() and c.tobytes() == d.tobytes()


# -------------------------------------------------------------- edge shapes

@pytest.mark.parametrize("n", [1, 3, 7, 8, 9, 255, 1023, 1025, 4099, 65537, (1 << 20) + 3])
@pytest.mark.parametrize("op", ["sum", "mean", "max", "argmax"])
def test_flat_ragged(hip, orc, n, op):
    x = SplitMix64(n).normal((n,), 0.0, 3.0)
    check(op, x, (n,), orc)


@pytest.mark.parametrize("op", ["sum", "max", "argmax"])
def test_flat_unaligned_pointer(hip, orc, op):
    x = SplitMix64(77).uniform((10001,), -1, 1)
    check(op, x, (x.size,), orc, ptr_offset_floats=1)


@pytest.mark.parametrize("sizes", [(7, 9, 1), (3, 1025, 1), (64, 131072, 1), (5, 33, 1),
                                   (1, 7, 3), (2, 5, 9), (1, 257, 33), (3, 64, 17),
                                   (2, 100, 1000), (4, 4, 4096), (1, 3000, 260)])
@pytest.mark.parametrize("op", ["sum", "mean", "max", "argmax"])
def test_axis_shapes(hip, orc, sizes, op):
    o, d, i = sizes
    x = SplitMix64(o * 1000003 + d * 101 + i).normal((o, d, i), 0.0, 2.0)
    check(op, x, sizes, orc)


@pytest.mark.parametrize("sizes", [(64, 2048, 1), (32, 8192, 1), (16, 16384, 1), (2, 4096, 2048), (1, 4096, 512)],
                         ids=lambda v: str(v))
@pytest.mark.parametrize("op", ["sum", "mean", "max", "argmax"])
def test_whole_row_and_chunk_forms(hip, orc, sizes, op):
    """Shapes that take the straight-line kernels: whole aligned rows of one
    load batch (2048, 8192 and 16384 floats: 4, 16 and -- for argmax's
    256-thread rows -- 4 to 16 float4 a thread) and column chunks of exactly
    256 rows over whole tiles, with two outer slices."""
    o, d, i = sizes
    x = SplitMix64(0x3A11 + o + d + i).uniform((o, d, i), -2.0, 2.0)
    check(op, x, sizes, orc)


def test_argmax_ties_first_index(hip, orc):
    x = np.zeros((6, 40), np.float32)
    x[1, [3, 17, 39]] = 5.0          # repeated maximum -> first one
    x[2, :] = -1.0                   # all equal -> 0
    x[3, [0, 39]] = 2.0
    x[4, 10:] = 7.0
    x[5, :] = -np.inf                # all -inf -> 0
    for sizes in [(6, 40, 1), (1, 6, 40)]:
        check("argmax", x, sizes, orc)
    check("argmax", x.ravel(), (x.size,), orc)


def test_max_minus_inf_semantics(hip, orc):
    # flat and row forms start from -FLT_MAX (reduce.cpp:206); the column
    # form starts from the first slice, so an all -inf column stays -inf
    x = np.full((4, 16), -np.inf, np.float32)
    x[1, 5] = 3.0
    row = gpu_reduce("max", x, (4, 16, 1))
    assert row[0] == np.float32(-np.finfo(np.float32).max) and row[1] == 3.0
    col = gpu_reduce("max", x, (1, 4, 16))
    assert col[0] == -np.inf and col[5] == 3.0
    check("max", x, (4, 16, 1), orc)
    check("max", x, (1, 4, 16), orc)


def test_flat_zero_elements(hip):
    z = DeviceArray((1,), np.float32)
    for op, want in [("sum", 0.0), ("max", -np.finfo(np.float32).max)]:
        call(f"cxm_reduce_{op}_flat_f32", None, z.ptr, 0, None)
        assert z.numpy()[0] == np.float32(want)
    call("cxm_reduce_mean_flat_f32", None, z.ptr, 0, None)
    assert np.isnan(z.numpy()[0])
    assert lib().cxm_reduce_argmax_flat_f32(None, z.ptr, 0, None) == E_INVALID


def test_engine_mirror_names(hip, orc):
    # the reference's call shape: reduce::sum(Xx, Xz, outer, dim, inner)
    x = SplitMix64(5).uniform((3, 50, 8), -1, 1)
    dx = DeviceArray.from_numpy(x)
    dz = DeviceArray((24,), np.float32)
    engine.reduce.max(dx, dz, 3, 50, 8)
    assert np.array_equal(dz.numpy(), orc.reduce_axis("max", x, 3, 50, 8))
    engine.reduce.sum(dx, dz, x.size)
    assert abs(dz.numpy()[0] - np.sum(x.astype(np.float64))) <= SUM_TOL * np.abs(x).sum()


def _wait_limit(polls):
    old = ctypes.c_uint(0)
    call("cxm_exchange_wait_limit", polls, ctypes.byref(old))
    return old.value


@pytest.mark.parametrize("n", [4096 * 4096, (1 << 20) + 3, 1000003])
@pytest.mark.parametrize("op", ["sum", "mean", "max", "min", "norm1", "norm2"])
def test_flat_recompute_is_bit_identical(hip, orc, n, op):
    """Flat reductions with 32-bit partials combine them in one reader
    workgroup that waits for tagged slots; a partial it does not see within
    the wait limit is recomputed from the input with the writer's arithmetic.
    Forcing that for every segment (limit 0) gives the same bits."""
    x = SplitMix64(0xF1A7 + n).uniform((n,), -1.0, 1.0)
    normal = gpu_reduce(op, x, (n,))
    old = _wait_limit(0)
    try:
        forced = gpu_reduce(op, x, (n,))
    finally:
        _wait_limit(old)
    assert normal.tobytes() == forced.tobytes()
    ref = orc.reduce_flat(op, x)
    if op in ("max", "min"):
        assert normal.tobytes() == ref.tobytes()
    else:
        assert abs(float(normal[0]) - float(ref[0])) <= SUM_TOL * max(float(np.abs(x).sum()), 1e-30)


def test_flat_slot_state_across_shapes(hip, orc):
    """Flat reductions of different lengths (different segment counts over
    the same tagged slots), interleaved with row, column and segmented-row
    reductions on the same stream, each checked against the oracle: no call
    reads a partial an earlier call left behind."""
    g = SplitMix64(0x51075)
    seq = [(1 << 24,), (100003,), (3, 50000, 1), (1 << 24,), (5000,), (1, 4096, 4096), ((1 << 22) + 1,),
           (1 << 24,), (777,), (1 << 21,)]
    for sizes in seq:
        x = g.uniform(sizes if len(sizes) > 1 else sizes[0], -1.0, 1.0)
        check("sum", x, sizes, orc)
        check("max", x, sizes, orc)


@pytest.mark.parametrize("off", [1, 2, 3])
@pytest.mark.parametrize("sizes", [((1 << 22) + 3,), (3, 100003, 1), (64, 4097, 1), (2, 5, 1)])
@pytest.mark.parametrize("op", ["sum", "max", "argmax"])
def test_unaligned_ragged_rows(hip, orc, off, sizes, op):
    """Row bases off 16-byte alignment and lengths not a multiple of 4: each
    row's head (before its first aligned float4) and tail are folded in by
    its first segment, the body still takes 128-bit loads."""
    x = SplitMix64(off * 7919 + sum(sizes)).normal(sizes if len(sizes) > 1 else sizes[0], 0.0, 2.0)
    check(op, x, sizes, orc, ptr_offset_floats=off)

