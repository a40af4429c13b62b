"""Pins the oracle's sgemv restatement (oracle/oracle.c, orc_sgemv_ld): the
reference's edge cases (tests/sgemv/edge-cases*.json, both layouts) against
numpy and hand values, random strided cases, reference BLAS's quick returns,
alpha = 0 and the no-transpose form's skipping of zero x entries
(tests/sgemv/src/test.sgemv.js:157-202, 299-387), and a planted mistake."""
import numpy as np
import pytest

from oracle import orc
from tests import refcases as rc


@pytest.mark.parametrize("routine", ["sgemv", "dgemv"])
@pytest.mark.parametrize("cm", [False, True])
def test_edge_cases_against_numpy(routine, cm):
    # dgemv (tests/dgemv/edge-cases*.json) runs the same restatement on doubles
    for c in rc.load(routine, cm):
        call = rc.gemv_call(c, np.float64)
        out, _ = orc.sgemv_ld(*call)
        assert np.array_equal(out, rc.numpy_gemv(*call)), c["label"]


def test_hand_values():
    # [[1,2,3],[4,5,6]] row-major: row sums (6, 15), column sums (5, 7, 9)
    rows = [c for c in rc.load("sgemv") if c["label"].startswith("NoTrans: row sums")][0]
    cols = [c for c in rc.load("sgemv") if c["label"].startswith("Trans: column sums")][0]
    assert list(orc.sgemv_ld(*rc.gemv_call(rows, np.float64))[0]) == [6.0, 15.0]
    assert list(orc.sgemv_ld(*rc.gemv_call(cols, np.float64))[0]) == [5.0, 7.0, 9.0]
    # incy = 2 leaves the gap: y = [2*3, 99]
    c = [c for c in rc.load("sgemv") if c["label"].startswith("incy=2")][0]
    assert list(orc.sgemv_ld(*rc.gemv_call(c, np.float64))[0]) == [6.0, 99.0]


@pytest.mark.parametrize("trans", [0, 1])
@pytest.mark.parametrize("inc", [1, 3])
def test_random_against_numpy(trans, inc):
    m, n, lda = 37, 23, 41
    A = orc.random_f32(lda * n, -1, 1, 1).astype(np.float64)
    xl, yl = (n, m) if trans == 0 else (m, n)
    x = orc.random_f32((xl - 1) * inc + 1, -1, 1, 2).astype(np.float64)
    y = orc.random_f32((yl - 1) * inc + 1, -1, 1, 3).astype(np.float64)
    call = (trans, m, n, 1.5, A, lda, x, inc, -0.5, y, inc)
    out, ad = orc.sgemv_ld(*call)
    ref = rc.numpy_gemv(*call)
    assert np.allclose(out, ref, rtol=1e-13, atol=1e-13)
    assert np.all(ad > 0)
    # planted mistake, on a square matrix: the transposed product must differ
    q = 29
    Aq = orc.random_f32(q * q, -1, 1, 4).astype(np.float64)
    xq = orc.random_f32((q - 1) * inc + 1, -1, 1, 5).astype(np.float64)
    yq = orc.random_f32((q - 1) * inc + 1, -1, 1, 6).astype(np.float64)
    sq = (trans, q, q, 1.5, Aq, q, xq, inc, -0.5, yq, inc)
    assert np.allclose(orc.sgemv_ld(*sq)[0], rc.numpy_gemv(*sq), rtol=1e-13, atol=1e-13)
    assert not np.allclose(orc.sgemv_ld(*sq)[0], rc.numpy_gemv(1 - trans, *sq[1:]), rtol=1e-6)


def test_quick_returns_and_alpha_zero():
    y = np.array([1.0, np.nan, 3.0])
    A = np.array([np.nan, np.inf, 1.0, 2.0, 3.0, 4.0])
    x = np.array([np.inf, 1.0, 2.0])
    # m == 0 / n == 0: y untouched (beta not applied)
    assert np.array_equal(orc.sgemv_ld(0, 3, 0, 1.5, A, 3, x, 1, 0.5, y, 1)[0], y, equal_nan=True)
    assert np.array_equal(orc.sgemv_ld(1, 0, 3, 1.5, A, 1, x, 1, 0.5, y, 1)[0], y, equal_nan=True)
    # alpha == 0, beta == 1: untouched; beta == 0: zeros (NaN cleared)
    assert np.array_equal(orc.sgemv_ld(0, 3, 2, 0.0, A, 3, x, 1, 1.0, y, 1)[0], y, equal_nan=True)
    assert np.array_equal(orc.sgemv_ld(0, 3, 2, 0.0, A, 3, x, 1, 0.0, y, 1)[0], np.zeros(3))
    out = orc.sgemv_ld(0, 3, 2, 0.0, A, 3, x, 1, 2.0, y, 1)[0]
    assert out[0] == 2.0 and np.isnan(out[1]) and out[2] == 6.0


def test_zero_x_entries_skip_their_column_only_without_transpose():
    # column 0 of A holds NaN and Inf; x[0] = 0
    A = np.array([np.nan, np.inf, 1.0, 2.0])  # 2 x 2 column-major
    x = np.array([0.0, 1.0])
    y = np.zeros(2)
    out, _ = orc.sgemv_ld(0, 2, 2, 1.0, A, 2, x, 1, 0.0, y, 1)
    assert list(out) == [1.0, 2.0]  # column 0 skipped
    out, _ = orc.sgemv_ld(1, 2, 2, 1.0, A, 2, x, 1, 0.0, y, 1)
    assert np.isnan(out[0]) and out[1] == 2.0  # dot form: 0 * NaN, 0 * Inf taken
