"""NaN and signed-zero semantics of the gfx950 max / min / argmax / argmin
(every form: flat, rows, columns; aligned, ragged and misaligned bases).

The rule the library states (include/cxm_hip.h, reductions):
  * max / min are IEEE 754-2019 maximum / minimum: NaN when any element is
    NaN; a +0/-0 tie gives +0 (max) or -0 (min).
  * argmax / argmin skip NaN elements, except a NaN first element of the
    row, column or flat array, which gives index 0; +0 and -0 compare equal,
    so the first of them wins.
The reference's _mm256_max_ps lane fold (Engine/AVX2/functions.hpp:314-325)
is position-dependent on these inputs, so the expected values here come
from that rule as tests/nan_rules.py restates it (checked on the CPU
against the reference's own argmax loop and a pairwise IEEE fold by
tests/test_nan_rules.py), not from the oracle.
"""
import numpy as np
import pytest

from cortexmind_amd._lib import call
from cortexmind_amd.data import SplitMix64
from cortexmind_amd.device import DeviceArray

from nan_rules import arg_rule, value_rule

pytestmark = pytest.mark.gpu


def run(op, x, sizes, off=0):
    flat = np.ascontiguousarray(x, np.float32).ravel()
    dx = DeviceArray.from_numpy(np.concatenate([np.zeros(off, np.float32), flat]))
    n_out = 1 if len(sizes) == 1 else sizes[0] * sizes[2]
    dz = DeviceArray((n_out,), np.int32 if op.startswith("arg") else np.float32)
    if len(sizes) == 1:
        call(f"cxm_reduce_{op}_flat_f32", dx.ptr + 4 * off, dz.ptr, sizes[0], None)
    else:
        call(f"cxm_reduce_{op}_f32", dx.ptr + 4 * off, dz.ptr, *sizes, None)
    return dz.numpy()


def slices(x, sizes):
    """The reduced slices as rows of a [slices, n] array, each in storage
    order along the reduced axis."""
    a = np.asarray(x, np.float32)
    if len(sizes) == 1:
        return a.reshape(1, -1)
    o, d, i = sizes
    return a.reshape(o, d, i).transpose(0, 2, 1).reshape(o * i, d)


def check(op, x, sizes, off=0):
    got = run(op, x, sizes, off)
    a = slices(x, sizes)
    if op.startswith("arg"):
        want = arg_rule(op, a)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, (op, sizes, off, bad[:5], got[bad[:5]], want[bad[:5]])
    else:
        rows = len(sizes) == 1 or sizes[2] == 1
        start = None if not rows else (-np.finfo(np.float32).max if op == "max" else np.finfo(np.float32).max)
        want = value_rule(op, a, start)
        same = (np.isnan(got) & np.isnan(want)) | (got.view(np.uint32) == want.view(np.uint32))
        bad = np.nonzero(~same)[0]
        assert bad.size == 0, (op, sizes, off, bad[:5], got[bad[:5]], want[bad[:5]])


def plant(g, shape, nan_frac=0.0, zero_tie=False, nan_first=False):
    """U(-1, 1) data; with zero_tie every element is <= 0 and a mix of +0
    and -0 is planted so that the max is a signed-zero tie (and -x for the
    min); NaNs at random positions; optionally a NaN first element."""
    x = g.uniform(shape, -1.0, 1.0).astype(np.float32)
    flat = x.reshape(-1)
    rng = np.random.default_rng(int(flat.size) + int(nan_frac * 1000) + zero_tie)
    if zero_tie:
        flat[:] = -np.abs(flat) - np.float32(0.5)
        idx = rng.choice(flat.size, size=max(4, flat.size // 500), replace=False)
        flat[idx] = np.where(rng.random(idx.size) < 0.5, np.float32(0.0), np.float32(-0.0))
    if nan_frac:
        idx = rng.choice(flat.size, size=max(1, int(flat.size * nan_frac)), replace=False)
        flat[idx] = np.nan
    if nan_first:
        flat[0] = np.nan
    return x


SHAPES = [(1 << 20,), ((1 << 20) + 37,), (5000,), (64, 4096, 1), (37, 1000, 1), (1, 4096, 4096),
          (3, 3000, 512), (2, 700, 301), (1, 513, 64)]


@pytest.mark.parametrize("sizes", SHAPES, ids=str)
@pytest.mark.parametrize("op", ["max", "min", "argmax", "argmin"])
def test_nan_scattered(hip, op, sizes):
    g = SplitMix64(0x7A00 + len(sizes) + sizes[0])
    x = plant(g, (int(np.prod(sizes)),), nan_frac=2e-4)
    check(op, x, sizes)


@pytest.mark.parametrize("sizes", SHAPES, ids=str)
@pytest.mark.parametrize("op", ["max", "min", "argmax", "argmin"])
def test_signed_zero_ties(hip, op, sizes):
    g = SplitMix64(0x7B00 + sizes[0])
    x = plant(g, (int(np.prod(sizes)),), zero_tie=True)
    if op in ("min", "argmin"):
        x = -x  # every element >= 0, the min a +0/-0 tie
    check(op, x, sizes)


@pytest.mark.parametrize("sizes", [(4097,), (64, 4096, 1), (37, 1000, 1), (1, 4096, 4096), (3, 3000, 512),
                                   (2, 700, 301)], ids=str)
@pytest.mark.parametrize("op", ["argmax", "argmin"])
def test_nan_first_element(hip, op, sizes):
    """A NaN first element of each row / column (and of the flat array) is
    the answer, index 0, whatever follows; also with more NaNs behind it."""
    g = SplitMix64(0x7C00 + sizes[0])
    x = plant(g, (int(np.prod(sizes)),), nan_frac=1e-3)
    if len(sizes) == 1:
        x[0] = np.nan
    else:
        o, d, i = sizes
        x.reshape(o, d, i)[:, 0, :] = np.nan
    check(op, x, sizes)


@pytest.mark.parametrize("op", ["max", "min", "argmax", "argmin"])
def test_all_nan_and_misaligned(hip, op):
    """All-NaN slices (max/min NaN, argmax/argmin 0) and bases 4 bytes past
    16-byte alignment (the head elements go through the scalar fold)."""
    g = SplitMix64(0x7D00)
    x = plant(g, (7 * 1000,), nan_frac=1e-3)
    x[:1000] = np.nan  # row 0 all NaN
    for off in (0, 1, 3):
        check(op, x, (7, 1000, 1), off)
        check(op, x, (7000,), off)
        check(op, x, (1, 7, 1000), off)
