"""The allocation-free lm-head entry point (e4b_k_q6k_gemv_argmax_noalloc)
against e4b_k_q6k_gemv_argmax, through the C-ABI.

Both run the same kernels (f32 -> f16 hi/lo split, Q6_K GEMV with per-block
argmax partials, the fold), so logits and argmax must be bit-identical.  Two
calls in a row, the second with a smaller, ragged input, check that the
scratch array left over from the first call does not leak into the second.
The argmax of the first call is also checked against the CPU oracle (ties:
either tied index, as in test_gemv_gpu.py).

The property the entry point exists for: it can be captured into a hipGraph.
A captured call replays (three times, with eager calls that overwrite the
scratch array in between) to the direct call's logits and argmax; in a fresh
process, whose workspace is still empty, the workspace entry point fails
inside a capture with E4B_EINVAL while the no-alloc one, called there for the
first time, captures and replays to the workspace entry point's result.
"""
import ctypes as C
import os
import subprocess
import sys

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


def _hip():
    """The HIP runtime's stream-capture and graph calls (test plumbing)."""
    try:
        h = C.CDLL("libamdhip64.so")
    except OSError:
        h = C.CDLL("/opt/rocm/lib/libamdhip64.so")
    vp, pp = C.c_void_p, C.POINTER(C.c_void_p)
    for name, args in (("hipStreamCreate", [pp]), ("hipStreamDestroy", [vp]), ("hipStreamSynchronize", [vp]),
                       ("hipStreamBeginCapture", [vp, C.c_int]), ("hipStreamEndCapture", [vp, pp]),
                       ("hipGraphInstantiate", [pp, vp, vp, C.c_char_p, C.c_size_t]),
                       ("hipGraphLaunch", [vp, vp]), ("hipGraphExecDestroy", [vp]), ("hipGraphDestroy", [vp])):
        f = getattr(h, name)
        f.argtypes, f.restype = args, C.c_int
    return h


def _ok(rc, what):
    assert rc == 0, f"{what} -> hipError {rc}"


def test_noalloc_lmhead_captured_into_a_graph_and_replayed():
    rows, cols, softcap = 4096, 2048, 30.0
    print(f"noalloc lm-head under capture {rows}x{cols}", flush=True)
    w = formats.synth_q6k(21, rows, cols, 1e-3)
    wd = DeviceBuffer.from_array(q6k_pack(w, rows, cols))
    xd = DeviceBuffer.from_array(formats.synth_normal(22, cols))
    xd2 = DeviceBuffer.from_array(formats.synth_normal(23, cols))
    fn = _lib.lib.e4b_k_q6k_gemv_argmax_noalloc
    want = _run("e4b_k_q6k_gemv_argmax_noalloc", wd, rows, cols, xd, softcap, True)
    other = _run("e4b_k_q6k_gemv_argmax_noalloc", wd, rows, cols, xd2, softcap, True)
    assert not np.array_equal(want[0], other[0])
    hip = _hip()
    st, g, ge = C.c_void_p(), C.c_void_p(), C.c_void_p()
    _ok(hip.hipStreamCreate(C.byref(st)), "hipStreamCreate")
    lg, am = DeviceBuffer(rows * 4), DeviceBuffer(8)
    _ok(hip.hipStreamBeginCapture(st, 1), "hipStreamBeginCapture")  # thread-local mode
    rc = fn(_vp(wd), rows, cols, _vp(xd), softcap, _vp(lg), _vp(am), st)
    _ok(hip.hipStreamEndCapture(st, C.byref(g)), "hipStreamEndCapture")
    _lib.check(rc, "e4b_k_q6k_gemv_argmax_noalloc (captured)")
    _ok(hip.hipGraphInstantiate(C.byref(ge), g, None, None, 0), "hipGraphInstantiate")
    for rep in range(3):
        lg.fill(0)
        am.fill(0)
        _ok(hip.hipGraphLaunch(ge, st), "hipGraphLaunch")
        _ok(hip.hipStreamSynchronize(st), "hipStreamSynchronize")
        a = am.download(np.uint32, 2)
        np.testing.assert_array_equal(lg.download(np.float32, rows), want[0])
        assert (int(a[0]), int(a[1])) == want[1:], f"replay {rep}"
        # eager work between replays: the same scratch array, another input
        got = _run("e4b_k_q6k_gemv_argmax_noalloc", wd, rows, cols, xd2, softcap, True)
        np.testing.assert_array_equal(got[0], other[0])
    for f, h in ((hip.hipGraphExecDestroy, ge), (hip.hipGraphDestroy, g), (hip.hipStreamDestroy, st)):
        _ok(f(h), f.__name__)
    for b in (wd, xd, xd2, lg, am):
        b.free()


_CHILD = r"""
import ctypes as C
import sys
import numpy as np
from e4b import _lib, formats
from e4b.device import DeviceBuffer
from e4b.formats import q6k_pack
from tests.test_zz_no_alloc import _hip, _ok, _vp
rows, cols = 2048, 1024
wd = DeviceBuffer.from_array(q6k_pack(formats.synth_q6k(31, rows, cols, 1e-3), rows, cols))
xd = DeviceBuffer.from_array(formats.synth_normal(32, cols))
hip = _hip()
st, g, ge = C.c_void_p(), C.c_void_p(), C.c_void_p()
_ok(hip.hipStreamCreate(C.byref(st)), "hipStreamCreate")
lg, am = DeviceBuffer(rows * 4), DeviceBuffer(8)
_ok(hip.hipStreamBeginCapture(st, 1), "hipStreamBeginCapture")
rc = _lib.lib.e4b_k_q6k_gemv_argmax(_vp(wd), rows, cols, _vp(xd), 0.0, _vp(lg), _vp(am), st)
err = _lib.last_error()
_ok(hip.hipStreamEndCapture(st, C.byref(g)), "hipStreamEndCapture")
print("workspace under capture:", rc, err, flush=True)
assert rc == _lib.E4B_EINVAL and "stream capture" in err
if g.value:
    hip.hipGraphDestroy(g)
g = C.c_void_p()
_ok(hip.hipStreamBeginCapture(st, 1), "hipStreamBeginCapture")
rc = _lib.lib.e4b_k_q6k_gemv_argmax_noalloc(_vp(wd), rows, cols, _vp(xd), 0.0, _vp(lg), _vp(am), st)
err = _lib.last_error()
_ok(hip.hipStreamEndCapture(st, C.byref(g)), "hipStreamEndCapture")
print("no-alloc, first call, under capture:", rc, err if rc else "", flush=True)
_lib.check(rc, "e4b_k_q6k_gemv_argmax_noalloc (captured first)")
_ok(hip.hipGraphInstantiate(C.byref(ge), g, None, None, 0), "hipGraphInstantiate")
_ok(hip.hipGraphLaunch(ge, st), "hipGraphLaunch")
_ok(hip.hipStreamSynchronize(st), "hipStreamSynchronize")
got = lg.download(np.float32, rows), am.download(np.uint32, 2)
lw, aw = DeviceBuffer(rows * 4), DeviceBuffer(8)
_lib.check(_lib.lib.e4b_k_q6k_gemv_argmax(_vp(wd), rows, cols, _vp(xd), 0.0, _vp(lw), _vp(aw), None), "workspace")
_lib.check(_lib.lib.e4b_sync(), "e4b_sync")
np.testing.assert_array_equal(got[0], lw.download(np.float32, rows))
np.testing.assert_array_equal(got[1], aw.download(np.uint32, 2))
print("CHILD OK", flush=True)
"""


def test_workspace_entry_fails_under_capture_in_a_fresh_process():
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([root, os.path.join(root, "e4b-webgpu_amd"),
                                                       os.environ.get("PYTHONPATH", "")]))
    print("fresh child: workspace and no-alloc lm-head under capture", flush=True)
    r = subprocess.run([sys.executable, "-c", _CHILD], cwd=root, env=env, capture_output=True, text=True,
                       timeout=110)
    print(r.stdout, r.stderr[-2000:])
    assert r.returncode == 0 and "CHILD OK" in r.stdout
