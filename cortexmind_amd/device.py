"""Device memory, streams and events over the C ABI (no torch).

DeviceArray is the Python counterpart of a tensor placed on the GPU: the
reference's Tensor::to(DeviceType::CUDA) allocates from the device pool and
uploads with a blocking copy (source/CortexMind/framework/Tensor/tensor.cpp:
151-171, Storage/storage.cpp:20-35, Memory/transform.cu:17-22); here
``DeviceArray.from_numpy`` does the same through cxm_dev_malloc and
cxm_memcpy_h2d, and ``numpy()`` is the download (cxm_memcpy_d2h).
"""
from __future__ import annotations

import atexit
import ctypes

import numpy as np

from ._lib import call, lib

_exiting = False


@atexit.register
def _mark_exit():
    # Device memory is returned with the process; freeing from finalizers
    # during interpreter shutdown would race the HIP runtime's own teardown.
    global _exiting
    _exiting = True


class Stream:
    """An owned non-blocking HIP stream (or the null stream when null=True)."""

    def __init__(self, null: bool = False):
        self.handle = ctypes.c_void_p(None)
        self._owned = not null
        if self._owned:
            call("cxm_stream_create", ctypes.byref(self.handle))

    def sync(self) -> None:
        call("cxm_stream_sync", self.handle)

    def close(self) -> None:
        if self._owned and self.handle.value:
            call("cxm_stream_destroy", self.handle)
            self.handle = ctypes.c_void_p(None)
            self._owned = False


class Event:
    def __init__(self):
        self.handle = ctypes.c_void_p(None)
        call("cxm_event_create", ctypes.byref(self.handle))

    def record(self, stream: Stream | None = None) -> None:
        call("cxm_event_record", self.handle, stream.handle if stream else None)

    def sync(self) -> None:
        call("cxm_event_sync", self.handle)

    def elapsed_ms(self, later: "Event") -> float:
        ms = ctypes.c_float(0.0)
        call("cxm_event_elapsed_ms", ctypes.byref(ms), self.handle, later.handle)
        return float(ms.value)

    def close(self) -> None:
        if self.handle.value:
            call("cxm_event_destroy", self.handle)
            self.handle = ctypes.c_void_p(None)


class DeviceArray:
    """A contiguous device buffer with a numpy dtype and shape.  With
    pool=True the memory comes from the library's stream-ordered caching
    allocator (cxm_pool_alloc on `stream`) instead of a direct allocation."""

    def __init__(self, shape, dtype=np.float32, pool: bool = False, stream: "Stream | None" = None):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.size = int(np.prod(self.shape)) if self.shape else 1
        self.nbytes = self.size * self.dtype.itemsize
        self._ptr = ctypes.c_void_p(None)
        self._pool = bool(pool)
        if self.nbytes:
            if self._pool:
                call("cxm_pool_alloc", ctypes.byref(self._ptr), self.nbytes, stream.handle if stream else None)
            else:
                call("cxm_dev_malloc", ctypes.byref(self._ptr), self.nbytes)

    @property
    def ptr(self) -> int | None:
        return self._ptr.value

    @classmethod
    def from_numpy(cls, a: np.ndarray, stream: Stream | None = None) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.upload(a, stream)
        return d

    def upload(self, a: np.ndarray, stream: Stream | None = None) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.size == self.size
        if self.nbytes:
            call("cxm_memcpy_h2d", self.ptr, a.ctypes.data, self.nbytes,
                 stream.handle if stream else None)
            # the copy reads host memory asynchronously: keep it alive until done
            if stream:
                stream.sync()
            else:
                call("cxm_device_sync")

    def numpy(self, stream: Stream | None = None) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            call("cxm_memcpy_d2h", out.ctypes.data, self.ptr, self.nbytes,
                 stream.handle if stream else None)
        return out

    def fill_bytes(self, byte_value: int = 0, stream: Stream | None = None) -> None:
        if self.nbytes:
            call("cxm_memset", self.ptr, int(byte_value), self.nbytes, stream.handle if stream else None)

    def free(self) -> None:
        if self._ptr.value:
            call("cxm_pool_free" if self._pool else "cxm_dev_free", self._ptr)
            self._ptr = ctypes.c_void_p(None)

    def __del__(self):
        try:
            if self._ptr.value and not _exiting:
                (lib().cxm_pool_free if self._pool else lib().cxm_dev_free)(self._ptr)
                self._ptr = ctypes.c_void_p(None)
        except Exception:
            pass


def device_count() -> int:
    n = ctypes.c_int(0)
    st = lib().cxm_device_count(ctypes.byref(n))
    return n.value if st == 0 else 0


def device_info() -> dict:
    name = ctypes.create_string_buffer(256)
    arch = ctypes.create_string_buffer(256)
    cus = ctypes.c_int(0)
    call("cxm_device_info", name, 256, ctypes.byref(cus), arch, 256)
    return {"name": name.value.decode(), "arch": arch.value.decode(), "cus": cus.value}


def pool_stats() -> dict:
    """The caching allocator's counters (cxm_pool_stats)."""
    from ._lib import PoolStats

    st = PoolStats()
    call("cxm_pool_stats", ctypes.byref(st))
    return {name: int(getattr(st, name)) for name, _ in PoolStats._fields_}


def pool_release() -> None:
    call("cxm_pool_release")
