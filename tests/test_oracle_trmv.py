"""Pins the oracle's strmv / dtrmv restatement (oracle/oracle.c,
orc_strmv_ld): the reference's edge cases (tests/{strmv,dtrmv}/edge-cases*.json,
both layouts) against numpy and hand values, random strided cases in both
triangles and both forms with the unstored triangle holding NaN (never
read), the unit diagonal never read, the column form's zero-x skip and the
dot form's lack of one (tests/strmv/src/test.strmv.js:258-306), and planted
mistakes (the layout flip of trans dropped, the diagonal read under unit)
that these checks reject."""
import numpy as np
import pytest

from oracle import orc
from tests import refcases as rc


def close(a, b, rel=1e-12):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return bool(np.all((a == b) | (np.abs(a - b) <= rel * np.maximum(np.abs(b), 1.0))))


@pytest.mark.parametrize("routine", ["strmv", "dtrmv"])
@pytest.mark.parametrize("cm", [False, True])
def test_edge_cases_against_numpy(routine, cm):
    for c in rc.load(routine, cm):
        call = rc.trmv_call(c, np.float64)
        out, _ = orc.strmv_ld(*call)
        assert np.array_equal(out, rc.numpy_trmv(*call)), c["label"]


def test_hand_values():
    # row-major [1, 99; 2, 3]: lower T = [[1, 0], [2, 3]], upper T = [[1, 2],
    # [0, 3]] (99 / the other corner never read); x = [1, 1]
    want = {"lower no-transpose": [1, 5], "upper no-transpose": [3, 3], "lower transpose": [3, 3],
            "upper transpose": [1, 5]}
    for c in rc.load("strmv"):
        if c["label"] in want:
            out, _ = orc.strmv_ld(*rc.trmv_call(c, np.float64))
            assert list(out[:2]) == want[c["label"]], c["label"]
            # planted: the layout flip of trans dropped reads T^T for T
            uplo, trans, *rest = rc.trmv_call(c, np.float64)
            wrong, _ = orc.strmv_ld(uplo, 1 - trans, *rest)
            assert list(wrong[:2]) != want[c["label"]]


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("trans", [0, 1])
@pytest.mark.parametrize("unit", [0, 1])
@pytest.mark.parametrize("n,inc", [(70, 1), (150, 3), (1, 2)])
def test_random_strided_unstored_nan(uplo, trans, unit, n, inc):
    lda = n + 2
    A = orc.random_f64(n * lda, -1, 1, 51)
    i, j = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
    unstored = (i < j) if uplo == 1 else (i > j)
    A[(i + j * lda)[unstored]] = np.nan
    if unit:
        A[np.arange(n) * (lda + 1)] = np.nan  # the diagonal is never read
    x = orc.random_f64((n - 1) * inc + 1, -1, 1, 52)
    y = orc.random_f64((n - 1) * inc + 1, -1, 1, 53)
    call = (uplo, trans, unit, n, A, lda, x, inc, y, inc)
    out, ad = orc.strmv_ld(*call)
    assert np.all(np.isfinite(out)) and close(out, rc.numpy_trmv(*call))
    gaps = np.ones(len(y), bool)
    gaps[np.arange(n) * inc] = False
    assert np.array_equal(out[gaps], y[gaps])
    assert np.all(ad[:n] >= np.abs(out[np.arange(n) * inc]) * (1 - 1e-12))
    if unit:
        # planted: the diagonal read under unit brings its NaN in
        wrong, _ = orc.strmv_ld(uplo, trans, 0, n, A, lda, x, inc, y, inc)
        assert np.isnan(wrong).any()


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("n", [7, 300])
def test_zero_x_skip_only_in_column_form(uplo, n):
    # test.strmv.js:258-306: Infinity off the diagonal and NaN on it in the
    # columns where x is zero; the column form (no transpose) never forms
    # 0 * Inf, the dot form (transpose) takes every term
    A = orc.random_f64(n * n, -1, 1, 1)
    x = orc.random_f64(n, -1, 1, 2)
    x[1] = x[n - 1] = 0.0
    A[1 + 1 * n] = np.nan
    if uplo == 1:
        A[3 + 1 * n] = np.inf
    else:
        A[0 + (n - 1) * n] = np.inf
    y = np.zeros(n)
    col, _ = orc.strmv_ld(uplo, 0, 0, n, A, n, x, 1, y, 1)
    dot, _ = orc.strmv_ld(uplo, 1, 0, n, A, n, x, 1, y, 1)
    assert np.all(np.isfinite(col)) and close(col, rc.numpy_trmv(uplo, 0, 0, n, A, n, x, 1, y, 1))
    assert np.isnan(dot[1])  # column 1 of T^T x meets NaN * 0
