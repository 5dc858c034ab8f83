"""Helpers shared by the GPU parity tests (imported by test modules only)."""
import numpy as np

from cortexmind_amd.device import DeviceArray


def dev(a, offset_floats=0):
    """Upload `a`; with offset_floats > 0 the returned pointer is misaligned
    by that many floats inside a larger buffer (the buffer is kept alive on
    the returned object)."""
    a = np.ascontiguousarray(a)
    if offset_floats == 0:
        return DeviceArray.from_numpy(a)
    buf = DeviceArray.from_numpy(np.concatenate([np.zeros(offset_floats, a.dtype), a.ravel()]))
    return _View(buf, offset_floats * a.dtype.itemsize, a.shape, a.dtype)


class _View:
    def __init__(self, base, byte_offset, shape, dtype):
        self.base, self.ptr, self.shape, self.dtype = base, base.ptr + byte_offset, shape, np.dtype(dtype)
        self.size = int(np.prod(shape))

    def numpy(self):
        full = self.base.numpy().view(np.uint8)
        off = self.ptr - self.base.ptr
        return full[off:off + self.size * self.dtype.itemsize].view(self.dtype).reshape(self.shape)


def empty(shape, dtype=np.float32, offset_floats=0):
    if offset_floats == 0:
        return DeviceArray(shape, dtype)
    return dev(np.zeros(shape, dtype), offset_floats)


def ulp_dist(a, b):
    """Units in the last place between float32 arrays (same-sign ordering)."""
    ai = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7FFFFFFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFFFFFF), bi)
    return np.abs(ai - bi)


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))
