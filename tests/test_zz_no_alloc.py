"""The allocation-free lm-head entry point (e4b_k_q6k_gemv_argmax_noalloc)
against e4b_k_q6k_gemv_argmax, through the C-ABI.

Both run the same kernels (f32 -> f16 hi/lo split, Q6_K GEMV with per-block
argmax partials, the fold), so logits and argmax must be bit-identical.  Two
calls in a row, the second with a smaller, ragged input, check that the
scratch array left over from the first call does not leak into the second.
The argmax of the first call is also checked against the CPU oracle (ties:
either tied index, as in test_gemv_gpu.py).
"""
import ctypes as C

import numpy as np
import pytest

import oracle as orc
from e4b import _lib, formats
from e4b.device import DeviceBuffer
from e4b.formats import q6k_pack
from tests.util import top2_margin

pytestmark = pytest.mark.gpu


def _vp(b):
    return C.c_void_p(b.ptr) if b is not None else None


def _run(fn, wd, rows, cols, xd, softcap, with_logits):
    lg = DeviceBuffer(rows * 4) if with_logits else None
    am = DeviceBuffer(8)
    rc = getattr(_lib.lib, fn)(_vp(wd), rows, cols, _vp(xd), softcap, _vp(lg), _vp(am), None)
    _lib.check(rc, fn)
    _lib.check(_lib.lib.e4b_sync(), "e4b_sync")
    a = am.download(np.uint32, 2)
    return (lg.download(np.float32, rows) if lg is not None else None), int(a[0]), int(a[1])


@pytest.mark.parametrize("order", ["noalloc_first", "workspace_first"])
def test_noalloc_lmhead_matches_workspace_entry_point(order):
    cases = [(8192, 2048, 5, 30.0, True), (1000, 1024, 6, 0.0, False)]  # second call smaller and ragged
    for rows, cols, seed, softcap, with_logits in cases:
        print(f"noalloc lm-head {rows}x{cols} seed={seed} softcap={softcap} logits={with_logits} ({order})",
              flush=True)
        w = formats.synth_q6k(seed, rows, cols, 1e-3)
        x = formats.synth_normal(seed + 77, cols)
        wd = DeviceBuffer.from_array(q6k_pack(w, rows, cols))
        xd = DeviceBuffer.from_array(x)
        fns = ["e4b_k_q6k_gemv_argmax_noalloc", "e4b_k_q6k_gemv_argmax"]
        if order == "workspace_first":
            fns.reverse()
        res = {fn: _run(fn, wd, rows, cols, xd, softcap, with_logits) for fn in fns}
        (lg_n, i_n, v_n), (lg_w, i_w, v_w) = res[fns[0]], res[fns[1]]
        if order == "workspace_first":
            (lg_n, i_n, v_n), (lg_w, i_w, v_w) = (lg_w, i_w, v_w), (lg_n, i_n, v_n)
        assert (i_n, v_n) == (i_w, v_w)
        if with_logits:
            np.testing.assert_array_equal(lg_n, lg_w)
            ref = orc.q6k_gemv(w, rows, cols, x, softcap)
            ridx, rval = orc.argmax(ref)
            tol_abs = 1e-5 * float(np.max(np.abs(ref)))
            if top2_margin(ref) > 2 * tol_abs:
                assert i_n == ridx
            else:
                assert abs(ref[i_n] - rval) <= 2 * tol_abs
        for b in (wd, xd):
            b.free()


def test_noalloc_lmhead_rejects_columns_beyond_its_scratch():
    # the size check runs before any device access
    dummy = C.c_void_p(16)
    rc = _lib.lib.e4b_k_q6k_gemv_argmax_noalloc(dummy, 128, 8192, dummy, 0.0, None, dummy, None)
    assert rc == _lib.E4B_ERANGE
    assert "4096-column maximum" in _lib.last_error()
