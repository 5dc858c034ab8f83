"""The stream-ordered caching allocator through the C ABI (cxm_pool_*):
reuse on the allocating stream, no reuse across streams, kernels reading and
writing pool memory, release, and argument errors.  The allocator's
bookkeeping is also tested on the host (tests/cpp/pool_core_test.cpp)."""
import ctypes

import numpy as np
import pytest

from cortexmind_amd import engine
from cortexmind_amd._lib import E_INVALID, call, lib
from cortexmind_amd.device import DeviceArray, Stream, pool_release, pool_stats

pytestmark = pytest.mark.gpu


def test_reuse_same_stream_and_not_across(hip):
    s1, s2 = Stream(), Stream()
    p = ctypes.c_void_p()
    call("cxm_pool_alloc", ctypes.byref(p), 3 << 20, s1.handle)   # class 4 MiB
    first = p.value
    call("cxm_pool_free", p)
    st0 = pool_stats()
    q = ctypes.c_void_p()
    call("cxm_pool_alloc", ctypes.byref(q), 4 << 20, s1.handle)
    assert q.value == first and pool_stats()["hits"] == st0["hits"] + 1
    r = ctypes.c_void_p()
    call("cxm_pool_alloc", ctypes.byref(r), 4 << 20, s2.handle)   # other stream: a different block
    assert r.value != first
    call("cxm_pool_free", q)
    call("cxm_pool_free", r)
    s1.close()
    s2.close()


def test_kernels_on_pool_memory(hip, orc):
    x = np.random.default_rng(1).normal(size=(300, 257)).astype(np.float32)
    dx = DeviceArray(x.shape, pool=True)
    dx.upload(x)
    dz = DeviceArray((300,), pool=True)
    engine.reduce.max(dx, dz, 300, 257, 1)
    assert np.array_equal(dz.numpy(), orc.reduce_axis("max", x, 300, 257, 1))
    before = pool_stats()
    dx.free()
    dz.free()
    after = pool_stats()
    assert after["bytes_in_use"] < before["bytes_in_use"] and after["bytes_cached"] > before["bytes_cached"]


def test_release_and_errors(hip):
    a = DeviceArray((1 << 20,), pool=True)
    a.free()
    assert pool_stats()["bytes_cached"] > 0
    pool_release()
    assert pool_stats()["bytes_cached"] == 0
    d = DeviceArray((16,))
    assert lib().cxm_pool_free(d.ptr) == E_INVALID          # not a pool pointer
    p = ctypes.c_void_p()
    assert lib().cxm_pool_alloc(ctypes.byref(p), 0, None) == E_INVALID
    assert lib().cxm_pool_alloc(None, 16, None) == E_INVALID
    assert lib().cxm_pool_free(None) == 0                    # freeing null is a no-op
