"""The no-allocation reduction entry point (cxm_reduce_sum_noalloc_f32)
against cxm_reduce_sum_f32, through the C ABI: the same kernels and plan,
so the same bits, on two calls in a row (the second on a smaller input,
after the first left its partials in the static region), plus the oracle's
1e-5 * sum|x| bar.  Collected last (test_zz_), so a failure here cannot hide
other tests from `pytest -x`."""
import numpy as np
import pytest

from cortexmind_amd._lib import E_INVALID, call, lib
from cortexmind_amd.data import SplitMix64
from cortexmind_amd.device import DeviceArray, pool_stats

pytestmark = pytest.mark.gpu


def run(fn, x, sizes):
    dx = DeviceArray.from_numpy(np.ascontiguousarray(x, np.float32).ravel())
    o, d, i = sizes
    dz = DeviceArray((o * i,), np.float32)
    call(fn, dx.ptr, dz.ptr, o, d, i, None)
    return dz.numpy()


def check(orc, x, sizes):
    got = run("cxm_reduce_sum_noalloc_f32", x, sizes)
    want = run("cxm_reduce_sum_f32", x, sizes)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), sizes
    ref = orc.reduce_axis("sum", x, *sizes)
    o, d, i = sizes
    tol = 1e-5 * np.abs(np.asarray(x, np.float64)).reshape(o, d, i).sum(axis=1).ravel()
    assert np.all(np.abs(got.astype(np.float64) - ref) <= tol + 1e-30), sizes


# (first call, second smaller call) per reduction form: the flat sum as one
# row of (1, n, 1), row sums with several segments per row, column sums
# with several row chunks per tile
PAIRS = [
    ((1, 4096 * 4096, 1), (1, 1000003, 1)),
    ((64, 131072, 1), (3, 50000, 1)),
    ((1, 4096, 4096), (2, 700, 300)),
]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_allocating_entry(hip, orc, first, second):
    for k, sizes in enumerate((first, second)):
        x = SplitMix64(0xA110C + k + sizes[1]).uniform(sizes, -1.0, 1.0)
        check(orc, x, sizes)


def _free_bytes():
    """hipMemGetInfo's free bytes, from the HIP runtime the library links."""
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so.7")
    free, total = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert hip.hipDeviceSynchronize() == 0
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_noalloc_allocates_nothing(hip):
    """Device free memory does not move across noalloc calls on a fresh
    stream (a flat sum, whose segments meet in tagged slots, and a
    segmented row sum, whose segments meet through a ticket), while the
    allocating entry point on another fresh stream takes its workspace for
    the segmented row sum (at least 8 MiB), which shows the measure can see
    an allocation."""
    from cortexmind_amd.device import Stream

    n = 1 << 22
    x = SplitMix64(9).uniform((n,), -1.0, 1.0)
    dx = DeviceArray.from_numpy(x)
    dz = DeviceArray((64,), np.float32)
    rows = (4, n // 4, 1)  # a few long rows: several segments per row, combined by ticket
    s1, s2 = Stream(), Stream()
    for sizes in [(1, n, 1), rows]:  # set-up on this device
        call("cxm_reduce_sum_noalloc_f32", dx.ptr, dz.ptr, *sizes, s1.handle)
    s1.sync()
    f0 = _free_bytes()
    for _ in range(3):
        for sizes in [(1, n, 1), rows]:
            call("cxm_reduce_sum_noalloc_f32", dx.ptr, dz.ptr, *sizes, s1.handle)
    s1.sync()
    f1 = _free_bytes()
    call("cxm_reduce_sum_f32", dx.ptr, dz.ptr, *rows, s2.handle)
    s2.sync()
    f2 = _free_bytes()
    assert f1 == f0, (f0, f1)
    assert f1 - f2 >= 8 << 20, (f1, f2)
    s1.close()
    s2.close()


def test_noalloc_rejects_bad_arguments(hip):
    z = DeviceArray((1,), np.float32)
    assert lib().cxm_reduce_sum_noalloc_f32(None, z.ptr, 1, 8, 1, None) == E_INVALID
    assert lib().cxm_reduce_sum_noalloc_f32(z.ptr, z.ptr, 1, 0, 1, None) == E_INVALID
