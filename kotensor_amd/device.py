"""Device buffers and streams owned by the host side, through the C ABI only.

A :class:`DeviceBuffer` plays the role of the Kotlin ``MemorySegment`` that holds
a device pointer returned by ``kt_dev_alloc``: the host owns it and frees it.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib


class Stream:
    """A HIP stream created by ``kt_stream_create``; ``Stream.null()`` is the null stream."""

    def __init__(self, handle=None, owned=False):
        self.handle = handle
        self._owned = owned

    @classmethod
    def create(cls) -> "Stream":
        h = ctypes.c_void_p()
        _lib.call("kt_stream_create", ctypes.byref(h))
        return cls(h.value, owned=True)

    @classmethod
    def null(cls) -> "Stream":
        return cls(None, owned=False)

    def synchronize(self) -> None:
        _lib.call("kt_stream_sync", self.handle)

    def destroy(self) -> None:
        if self._owned and self.handle:
            _lib.call("kt_stream_destroy", self.handle)
        self.handle = None
        self._owned = False

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


_NULL = Stream.null()


def default_stream() -> Stream:
    return _NULL


class DeviceBuffer:
    """``nbytes`` of device memory from ``kt_dev_alloc``."""

    def __init__(self, nbytes: int):
        if nbytes < 0:
            raise _lib.IllegalArgumentException(f"negative size {nbytes}")
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        _lib.call("kt_dev_alloc", ctypes.c_size_t(self.nbytes), ctypes.byref(p))
        self._ptr = p.value

    @property
    def ptr(self) -> int | None:
        return self._ptr

    @classmethod
    def from_numpy(cls, array: np.ndarray, stream: Stream | None = None) -> "DeviceBuffer":
        array = np.ascontiguousarray(array)
        buf = cls(array.nbytes)
        buf.upload(array, stream)
        return buf

    def upload(self, array: np.ndarray, stream: Stream | None = None, offset: int = 0) -> None:
        array = np.ascontiguousarray(array)
        if offset + array.nbytes > self.nbytes:
            raise _lib.IllegalArgumentException(f"{array.nbytes} bytes do not fit at {offset} in {self.nbytes}")
        if array.nbytes:
            _lib.call("kt_memcpy_h2d", ctypes.c_void_p(self._ptr + offset), array.ctypes.data_as(ctypes.c_void_p),
                      ctypes.c_size_t(array.nbytes), (stream or _NULL).handle)

    def download(self, dtype, count: int | None = None, stream: Stream | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        if out.nbytes:
            if offset + out.nbytes > self.nbytes:
                raise _lib.IllegalArgumentException(f"{out.nbytes} bytes at {offset} exceed {self.nbytes}")
            _lib.call("kt_memcpy_d2h", out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(self._ptr + offset),
                      ctypes.c_size_t(out.nbytes), (stream or _NULL).handle)
        return out

    def copy_from(self, other: "DeviceBuffer", stream: Stream | None = None) -> None:
        n = min(self.nbytes, other.nbytes)
        if n:
            _lib.call("kt_memcpy_d2d", self._ptr, other.ptr, ctypes.c_size_t(n), (stream or _NULL).handle)

    def fill_zero(self, stream: Stream | None = None) -> None:
        if self.nbytes:
            _lib.call("kt_memset", self._ptr, 0, ctypes.c_size_t(self.nbytes), (stream or _NULL).handle)

    def free(self) -> None:
        if self._ptr:
            _lib.call("kt_dev_free", self._ptr)
        self._ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def synchronize(stream: Stream | None = None) -> None:
    (stream or _NULL).synchronize()


def device_count() -> int:
    n = ctypes.c_int32()
    _lib.call("kt_device_count", ctypes.byref(n))
    return n.value
