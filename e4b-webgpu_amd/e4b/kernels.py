"""Kernel-level entry points (parity tests and per-config benches).

Each wrapper takes DeviceBuffers and calls the matching C-ABI function; the
weights are device copies of the packed layouts from formats.py.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import DT_F16, DT_F32, check, lib
from .device import DeviceBuffer
from .formats import q40_pack, q6k_pack


def _vp(x) -> C.c_void_p:
    if x is None:
        return C.c_void_p(0)
    return C.c_void_p(x.ptr if isinstance(x, DeviceBuffer) else int(x))


class Q40Matrix:
    """A q4_0 matrix resident on the device in the library's packed layout."""

    def __init__(self, ggml: np.ndarray, rows: int, cols: int):
        self.rows, self.cols = rows, cols
        self.buf = DeviceBuffer.from_array(q40_pack(ggml, rows, cols))

    def gemv_dev(self, x: DeviceBuffer, x_dtype: int, y: DeviceBuffer, stream=None) -> None:
        check(lib.e4b_k_q40_gemv(_vp(self.buf), self.rows, self.cols, _vp(x), x_dtype, _vp(y), _vp(stream)),
              "e4b_k_q40_gemv")

    def gemv(self, x: np.ndarray) -> np.ndarray:
        """Host convenience: x is float32 or float16 [cols] -> float32 [rows]."""
        dt = DT_F16 if x.dtype == np.float16 else DT_F32
        xd = DeviceBuffer.from_array(x.astype(np.float16 if dt == DT_F16 else np.float32))
        yd = DeviceBuffer(self.rows * 4)
        self.gemv_dev(xd, dt, yd)
        return yd.download(np.float32, self.rows)


class Q6KMatrix:
    """A Q6_K matrix resident on the device in the library's packed layout."""

    def __init__(self, ggml: np.ndarray, rows: int, cols: int):
        self.rows, self.cols = rows, cols
        self.buf = DeviceBuffer.from_array(q6k_pack(ggml, rows, cols))

    def gemv_argmax_dev(self, x: DeviceBuffer, softcap: float, logits: DeviceBuffer | None,
                        amax: DeviceBuffer, stream=None) -> None:
        check(lib.e4b_k_q6k_gemv_argmax(_vp(self.buf), self.rows, self.cols, _vp(x), softcap, _vp(logits),
                                        _vp(amax), _vp(stream)), "e4b_k_q6k_gemv_argmax")

    def gemv_argmax(self, x: np.ndarray, softcap: float = 0.0):
        xd = DeviceBuffer.from_array(x.astype(np.float32))
        lg = DeviceBuffer(self.rows * 4)
        am = DeviceBuffer(8)
        self.gemv_argmax_dev(xd, softcap, lg, am)
        a = am.download(np.uint32, 2)
        return lg.download(np.float32, self.rows), int(a[0]), float(a[1:2].view(np.float32)[0])

    def row(self, r: int, mult: float = 1.0) -> np.ndarray:
        out = DeviceBuffer(self.cols * 4)
        check(lib.e4b_k_q6k_row(_vp(self.buf), self.rows, self.cols, r, mult, _vp(out), None), "e4b_k_q6k_row")
        return out.download(np.float32, self.cols)


def argmax(x: np.ndarray):
    xd = DeviceBuffer.from_array(np.ascontiguousarray(x, dtype=np.float32))
    am = DeviceBuffer(8)
    check(lib.e4b_k_argmax(_vp(xd), x.size, _vp(am), None), "e4b_k_argmax")
    a = am.download(np.uint32, 2)
    return int(a[0]), float(a[1:2].view(np.float32)[0])
