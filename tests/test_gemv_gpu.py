"""GPU parity of the dequant-GEMV kernels against the CPU oracle (configs c0, c1).

Tolerances (floating point): GEMV outputs within 1e-5 of max|y_oracle|
(the oracle accumulates in double; the kernels in f32 with exact products).
Integer outputs (argmax index) must match bit-exactly unless the oracle's
top-2 margin is below the logit tolerance, in which case the case is reported
as a near-tie and either tied index is accepted.
"""
import numpy as np
import pytest

import oracle as orc
from e4b import formats
from e4b.device import DeviceBuffer
from e4b.kernels import Q40Matrix, Q6KMatrix, argmax
from tests.util import max_rel_err, top2_margin

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-5


def test_fdot2_subnormal_pairs_exact():
    # every nibble value against x = +-1, +-2^-14 (f16 min normal), 1000: the
    # v_dot2 subnormal trick must give exactly (n - 8) * d * x
    rows, cols = 16, 32
    blocks = bytearray()
    for r in range(rows):
        blocks += np.float16(1.0).tobytes() + bytes([(r & 15) | ((r & 15) << 4)] * 16)
    w = np.frombuffer(bytes(blocks), np.uint8)
    M = Q40Matrix(w, rows, cols)
    for xv in (1.0, -1.0, 2.0 ** -14, 1000.0, 0.5):
        x = np.full(cols, xv, np.float16)
        y = M.gemv(x)
        want = np.array([(r - 8) * 32 * float(np.float16(xv)) for r in range(rows)], np.float32)
        np.testing.assert_array_equal(y, want)


@pytest.mark.parametrize("seed", [0, 1])
def test_q40_gemv_c0_f32(seed):
    rows, cols = 16384, 2048  # benchmark config c0
    w = formats.synth_q40(seed, rows, cols, 0.02)
    x = formats.synth_normal(1000 + seed, cols)
    y = Q40Matrix(w, rows, cols).gemv(x)
    ref = orc.q40_gemv(w, rows, cols, x)
    err = max_rel_err(y, ref)
    print(f"c0 seed={seed} max_rel_err={err:.3e}")
    assert err < GEMV_TOL


@pytest.mark.parametrize("rows,cols", [
    (3072, 2048), (2048, 2048), (32768, 2048), (2048, 16384), (256, 2048), (2048, 256),
    (8960, 2048), (1408, 2816), (2816, 704), (4224, 2816), (2816, 2112), (37, 96), (1, 32), (5, 6144),
])
def test_q40_gemv_shapes_f16(rows, cols):
    w = formats.synth_q40(rows * 7 + cols, rows, cols, 0.02)
    x = formats.synth_normal(rows + cols, cols).astype(np.float16)
    y = Q40Matrix(w, rows, cols).gemv(x)
    ref = orc.q40_gemv(w, rows, cols, x.astype(np.float32))
    err = max_rel_err(y, ref)
    assert err < GEMV_TOL, (rows, cols, err)


def test_q40_gemv_prepared_split_matches_f32():
    rows, cols = 512, 2048
    w = formats.synth_q40(5, rows, cols)
    x = formats.synth_normal(6, cols)
    M = Q40Matrix(w, rows, cols)
    xd = DeviceBuffer.from_array(x)
    hl = DeviceBuffer(cols * 4)
    from e4b._lib import DT_F32, DT_F32_HL, check, lib
    import ctypes as C
    check(lib.e4b_split_f32(C.c_void_p(xd.ptr), cols, C.c_void_p(hl.ptr), None), "split")
    # the device split is bit-identical to hi = f16(x), lo = f16(x - hi) (RNE)
    got = hl.download(np.uint16)
    hi = x.astype(np.float16)
    lo = (x - hi.astype(np.float32)).astype(np.float16)
    np.testing.assert_array_equal(got[:cols], hi.view(np.uint16))
    np.testing.assert_array_equal(got[cols:], lo.view(np.uint16))
    y1, y2 = DeviceBuffer(rows * 4), DeviceBuffer(rows * 4)
    M.gemv_dev(xd, DT_F32, y1)
    M.gemv_dev(hl, DT_F32_HL, y2)
    np.testing.assert_array_equal(y1.download(np.float32), y2.download(np.float32))


def _check_lmhead(rows, cols, seed, softcap):
    w = formats.synth_q6k(seed, rows, cols, 1e-3)
    x = formats.synth_normal(seed + 77, cols)
    lg, idx, val = Q6KMatrix(w, rows, cols).gemv_argmax(x, softcap)
    ref = orc.q6k_gemv(w, rows, cols, x, softcap)
    err = max_rel_err(lg, ref)
    ridx, rval = orc.argmax(ref)
    margin = top2_margin(ref)
    tol_abs = GEMV_TOL * float(np.max(np.abs(ref)))
    print(f"lmhead {rows}x{cols} seed={seed} err={err:.3e} idx gpu={idx} ref={ridx} margin={margin:.3e}")
    assert err < GEMV_TOL
    assert val == lg[idx]
    assert idx == int(np.argmax(lg))  # kernel argmax == argmax of its own logits (lowest index on ties)
    if margin > 2 * tol_abs:
        assert idx == ridx
    else:
        assert abs(ref[idx] - rval) <= 2 * tol_abs  # near-tie: either tied index


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_q6k_lmhead_argmax_c1(seed):
    _check_lmhead(262144, 2048, seed, 30.0)  # benchmark config c1


@pytest.mark.parametrize("rows,cols", [(1000, 256), (4099, 2816 // 256 * 256), (77, 4096)])
def test_q6k_lmhead_shapes(rows, cols):
    _check_lmhead(rows, cols, rows, 0.0)


def test_q6k_row_dequant():
    rows, cols = 300, 2048
    w = formats.synth_q6k(3, rows, cols)
    M = Q6KMatrix(w, rows, cols)
    for r in (0, 1, 129, 299):
        got = M.row(r, float(np.sqrt(2048)))
        want = orc.q6k_row(w, cols, r, float(np.sqrt(2048)))
        np.testing.assert_allclose(got, want, rtol=3e-7, atol=0)


def test_argmax_ties_nan_and_empty_like():
    x = formats.synth_normal(9, 262144)
    x[[17, 100000, 200000]] = 9.0
    assert argmax(x) == (17, 9.0)
    x[3] = np.nan
    assert argmax(x)[0] == 17
    x = np.full(70000, -np.inf, np.float32)
    assert argmax(x) == (0, float(np.float32(-3.0e38)))
    x = formats.synth_normal(10, 1000)
    assert argmax(x)[0] == orc.argmax(x)[0]


# --------------------------------------------------------------------------
# gate/up + GeGLU (kernels/q40gu.wgsl), plain and with the fused residual +
# RMSNorm prologue the decode step uses (kernels/rmsacc3.wgsl folded in).
# Output f16: within GEGLU_TOL of |want| plus 1e-4 of max|want| (one f16
# rounding of the product, GEMV error ~1e-6).
# --------------------------------------------------------------------------
GEGLU_TOL = 1.5e-3


def _geglu_want(w, ff, cols, x16):
    g = orc.q40_gemv(w, 2 * ff, cols, x16.astype(np.float32)).astype(np.float64)
    gate, up = g[:ff], g[ff:]
    gl = np.array([orc.gelu_tanh(float(v)) for v in gate])
    return gl * up


def _check_geglu(got, want, name):
    got = got.astype(np.float64)
    scale = np.abs(want).max()
    err = np.abs(got - want) - (GEGLU_TOL * np.abs(want) + 1e-4 * scale)
    print(f"{name}: max excess {err.max():.3e} (scale {scale:.3f})")
    assert err.max() <= 0


@pytest.mark.parametrize("ff,cols", [(16384, 2048), (704, 2816), (1000, 256)])
def test_q40_geglu(ff, cols):
    w = formats.synth_q40(ff + cols, 2 * ff, cols, 0.02)
    x = formats.synth_normal(7, cols).astype(np.float16)
    got = Q40Matrix(w, 2 * ff, cols).geglu(x)
    _check_geglu(got, _geglu_want(w, ff, cols, x), f"geglu {ff}x{cols}")


@pytest.mark.parametrize("ff,cols,with_resid", [(16384, 2048, True), (512, 256, True), (512, 1024, False)])
def test_q40_geglu_prenorm(ff, cols, with_resid):
    rng = np.random.default_rng(ff + cols)
    w = formats.synth_q40(3 * ff + cols, 2 * ff, cols, 0.02)
    h_in = rng.standard_normal(cols).astype(np.float32)
    resid = (3.0 * rng.standard_normal(cols)).astype(np.float32) if with_resid else None
    w_resid = (1.0 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    w_in = (1.0 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    scale = 0.75
    h_got, got = Q40Matrix(w, 2 * ff, cols).geglu_prenorm(h_in, resid, w_resid if with_resid else None, w_in, scale)
    h_want = h_in.astype(np.float64)
    if with_resid:
        h_want = h_want + orc.rmsnorm(resid, w_resid).astype(np.float64)
    h_want = h_want * scale
    np.testing.assert_allclose(h_got, h_want, rtol=2e-6, atol=2e-6 * np.abs(h_want).max())
    x16 = orc.rmsnorm(h_want.astype(np.float32), w_in).astype(np.float16)
    _check_geglu(got, _geglu_want(w, ff, cols, x16), f"geglu prenorm {ff}x{cols}")


def test_q40_geglu_prenorm_rejects_unsupported_hidden():
    from e4b._lib import E4BError
    w = formats.synth_q40(1, 2 * 64, 2816, 0.02)
    with pytest.raises(E4BError):
        Q40Matrix(w, 128, 2816).geglu_prenorm(np.zeros(2816, np.float32), None, None, np.ones(2816, np.float32))
