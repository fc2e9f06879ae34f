"""GPU parity of the batched q4_0 GEMM on the matrix cores (the prefill
GEMM) against the CPU oracle.

Reference: the oracle's q4_0 dequant (pinned in test_oracle.py) as a float64
matrix, Y_ref = X W^T in float64 with X the same f16 activations.  The
kernel's products (n - 8) x are exact in the f16 MFMA with f32 accumulation
and each block is scaled by its f32 scale, so the only difference is the f32
summation order: outputs within GEMM_TOL of max|Y_ref| per case.  The GeGLU
epilogue adds one f16 rounding: within GEGLU_TOL of |want| plus 1e-4 of
max|want|, as the GEMV tests.  Shapes cover every engine matrix at prefill
widths, ragged token counts (not multiples of 32 or of the 128-token tile),
ragged rows and a single token.
"""
import numpy as np
import pytest

import oracle as orc
from e4b import formats
from e4b.kernels import Q40Matrix
from tests.util import max_rel_err

pytestmark = pytest.mark.gpu

GEMM_TOL = 1e-5
GEGLU_TOL = 1.5e-3


def _w_dense(w, rows, cols):
    return orc.q40_dequant(w).astype(np.float64).reshape(rows, cols)


@pytest.mark.parametrize("rows,cols,m", [
    (3072, 2048, 512), (2048, 2048, 37), (256, 2048, 1), (2048, 256, 129), (8960, 2048, 64),
    (2048, 16384, 100), (37, 96, 33), (1408, 2816, 200), (2816, 704, 5), (4224, 2816, 31),
])
def test_q40_gemm(rows, cols, m):
    w = formats.synth_q40(rows * 3 + cols + m, rows, cols, 0.02)
    x = formats.synth_normal(rows + cols + m, m * cols).reshape(m, cols).astype(np.float16)
    got = Q40Matrix(w, rows, cols).gemm(x)
    ref = x.astype(np.float64) @ _w_dense(w, rows, cols).T
    err = max_rel_err(got.ravel(), ref.ravel())
    print(f"gemm {rows}x{cols} m={m}: max err {err:.3e} of max {np.abs(ref).max():.3f}")
    assert err < GEMM_TOL


def test_q40_gemm_matches_gemv_columns():
    # every token column against the decode GEMV on the same weights (both
    # are exact-product, f32-accumulated; they differ in summation order only)
    rows, cols, m = 512, 2048, 48
    w = formats.synth_q40(91, rows, cols, 0.02)
    x = formats.synth_normal(92, m * cols).reshape(m, cols).astype(np.float16)
    M = Q40Matrix(w, rows, cols)
    got = M.gemm(x)
    for t in (0, 1, 31, 32, 47):
        ref = M.gemv(x[t])
        assert max_rel_err(got[t], ref) < GEMM_TOL


@pytest.mark.parametrize("ff,cols,m", [(16384, 2048, 64), (704, 2816, 77), (1000, 256, 3)])
def test_q40_gemm_geglu(ff, cols, m):
    w = formats.synth_q40(ff + cols + m, 2 * ff, cols, 0.02)
    x = formats.synth_normal(ff + m, m * cols).reshape(m, cols).astype(np.float16)
    got = Q40Matrix(w, 2 * ff, cols).gemm_geglu(x).astype(np.float64)
    g = x.astype(np.float64) @ _w_dense(w, 2 * ff, cols).T
    gate, up = g[:, :ff], g[:, ff:]
    want = np.vectorize(orc.gelu_tanh)(gate) * up
    scale = np.abs(want).max()
    excess = np.abs(got - want) - (GEGLU_TOL * np.abs(want) + 1e-4 * scale)
    print(f"gemm geglu {ff}x{cols} m={m}: max excess {excess.max():.3e} (scale {scale:.3f})")
    assert excess.max() <= 0
