"""Device memory through the C ABI (replaces src/gpu.js:26-50 upload/alloc/readback)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import check, lib


def device_count() -> int:
    n = C.c_int(0)
    check(lib.e4b_device_count(C.byref(n)), "e4b_device_count")
    return n.value


def sync() -> None:
    check(lib.e4b_sync(), "e4b_sync")


class DeviceBuffer:
    """An owned device allocation.  ``ptr`` is the raw device address."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = lib.e4b_dev_alloc(max(self.nbytes, 1))
        if not p:
            check(-2, f"e4b_dev_alloc({self.nbytes})")
        self.ptr = int(p)

    @classmethod
    def from_array(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        if offset + arr.nbytes > self.nbytes:
            raise ValueError(f"upload of {arr.nbytes} B at {offset} overflows a {self.nbytes} B buffer")
        check(lib.e4b_memcpy_h2d(C.c_void_p(self.ptr + offset), arr.ctypes.data_as(C.c_void_p), arr.nbytes),
              "e4b_memcpy_h2d")

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download overflows the buffer")
        check(lib.e4b_memcpy_d2h(out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr + offset), out.nbytes),
              "e4b_memcpy_d2h")
        return out

    def fill(self, value: int = 0) -> None:
        check(lib.e4b_memset_dev(C.c_void_p(self.ptr), value, self.nbytes), "e4b_memset_dev")

    def free(self) -> None:
        if self.ptr:
            lib.e4b_dev_free(C.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    """A HIP event on the library's stream (NULL = the HIP null stream)."""

    def __init__(self):
        p = lib.e4b_event_create()
        if not p:
            check(-3, "e4b_event_create")
        self.ptr = int(p)

    def record(self, stream=None) -> None:
        check(lib.e4b_event_record(C.c_void_p(self.ptr), C.c_void_p(stream or 0)), "e4b_event_record")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0)
        check(lib.e4b_event_elapsed_ms(C.c_void_p(self.ptr), C.c_void_p(end.ptr), C.byref(ms)),
              "e4b_event_elapsed_ms")
        return float(ms.value)

    def __del__(self):
        try:
            lib.e4b_event_destroy(C.c_void_p(self.ptr))
        except Exception:
            pass
