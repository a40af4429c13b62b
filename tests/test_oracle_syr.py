"""Pins the oracle's ssyr / ssyr2 restatement (oracle/oracle.c, orc_ssyr2_ld;
dsyr / dsyr2 run it on doubles): the reference's edge cases
(tests/{ssyr,ssyr2,dsyr,dsyr2}/edge-cases*.json, both layouts) against numpy
and hand values, random strided cases in both triangles with lda padding,
the quick returns (n or alpha zero, vectors unread), the zero-entry column
skip (syr2: both entries zero), the untouched other triangle, and planted
mistakes (the full matrix updated, the rank-2 term dropped) that these checks
reject (tests/ssyr/src/test.ssyr.js:111-230, test.ssyr2.js:142-283)."""
import numpy as np
import pytest

from oracle import orc
from tests import refcases as rc


def close(a, b, rel=1e-13):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    same = (a == b) | (np.isnan(a) & np.isnan(b))
    return bool(np.all(same | (np.abs(a - b) <= rel * np.maximum(np.abs(b), 1.0))))


def run(call):
    if len(call) == 7:
        return orc.ssyr_ld(*call)
    return orc.ssyr2_ld(*call)


def numpy_ref(call):
    if len(call) == 7:
        uplo, n, alpha, x, incx, A, lda = call
        return rc.numpy_syr2(uplo, n, alpha, x, incx, None, 1, A, lda)
    return rc.numpy_syr2(*call)


@pytest.mark.parametrize("routine", ["ssyr", "ssyr2", "dsyr", "dsyr2"])
@pytest.mark.parametrize("cm", [False, True])
def test_edge_cases_against_numpy(routine, cm):
    for c in rc.load(routine, cm):
        call = rc.syr_call(c, np.float64)
        assert np.array_equal(run(call), numpy_ref(call)), c["label"]


def test_hand_values():
    # ssyr lower, x = [1, 2]: x x^T = [[1, 2], [2, 4]]; row-major lower is
    # column-major upper, so A = [a00 a01; a10 a11] row-major gets a01 = 0
    c = [c for c in rc.load("ssyr") if c["label"].startswith("lower")][0]
    A0 = np.array(c["A"], np.float64)
    got = orc.ssyr_ld(*rc.syr_call(c, np.float64))
    assert got[0] == A0[0] + 1 and got[2] == A0[2] + 2 and got[3] == A0[3] + 4 and got[1] == A0[1]
    # ssyr2 lower, x = [1, 2], y = [3, 4]: x y^T + y x^T = [[6, 10], [10, 16]]
    c = [c for c in rc.load("ssyr2") if c["label"].startswith("lower")][0]
    A0 = np.array(c["A"], np.float64)
    got = orc.ssyr2_ld(*rc.syr_call(c, np.float64))
    assert got[0] == A0[0] + 6 and got[2] == A0[2] + 10 and got[3] == A0[3] + 16 and got[1] == A0[1]


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("two", [False, True])
@pytest.mark.parametrize("n,inc,pad", [(70, 1, 3), (150, 3, 0), (1, 2, 4)])
def test_random_strided(uplo, two, n, inc, pad):
    lda = n + pad
    x = orc.random_f64((n - 1) * inc + 1, -1, 1, 301)
    y = orc.random_f64((n - 1) * inc + 1, -1, 1, 302) if two else None
    A = orc.random_f64(n * lda, -1, 1, 303)
    call = (uplo, n, 1.5, x, inc, y, inc, A, lda)
    got = orc.ssyr2_ld(*call)
    assert close(got, rc.numpy_syr2(*call))
    i, j = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
    tri = (i >= j) if uplo == 1 else (i <= j)
    idx = (i + j * lda)[tri]
    keep = np.ones(len(A), bool)
    keep[idx] = False
    assert np.array_equal(got[keep], A[keep])  # other triangle and padding untouched
    if n == 1:
        return  # one element: the triangle is the whole matrix
    # planted: the full matrix updated
    full = A.copy()
    xv, yv = x[np.arange(n) * inc], (y[np.arange(n) * inc] if two else x[np.arange(n) * inc])
    upd = 1.5 * (np.outer(xv, yv) + (np.outer(yv, xv) if two else 0))
    full[(i + j * lda).ravel()] += upd.ravel()
    assert not close(got, full)


def test_rank2_term_needed():
    n = 5
    x, y, A = orc.random_f64(n, -1, 1, 1), orc.random_f64(n, -1, 1, 2), np.zeros(n * n)
    got = orc.ssyr2_ld(1, n, 1.0, x, 1, y, 1, A, n).reshape(n, n).T
    want = np.tril(np.outer(x, y) + np.outer(y, x))
    assert np.allclose(got, want, rtol=1e-15)
    assert not np.allclose(got, np.tril(np.outer(x, y)))


def test_quick_returns_and_skips():
    n = 6
    A = orc.random_f64(n * n, -1, 1, 3)
    nan = np.full(n, np.nan)
    assert np.array_equal(orc.ssyr_ld(1, 6, 0.0, nan, 1, A, n), A)
    assert np.array_equal(orc.ssyr2_ld(2, 0, 1.5, nan, 1, nan, 1, A, n), A)
    x = orc.random_f64(n, -1, 1, 1)
    y = orc.random_f64(n, -1, 1, 2)
    x[[0, 3]] = 0.0
    y[[1, 3]] = 0.0
    x[1], y[5] = np.inf, np.nan
    g1 = orc.ssyr_ld(1, n, 1.5, x, 1, A, n).reshape(n, n).T
    Am = A.reshape(n, n).T
    assert np.array_equal(g1[:, 0], Am[:, 0]) and np.array_equal(g1[:, 3], Am[:, 3])  # x[j] = 0
    assert np.isinf(g1[1, 1]) and np.isnan(g1[3, 1])  # Inf * (alpha Inf); 0 * Inf in column 1
    g2 = orc.ssyr2_ld(1, n, 1.5, x, 1, y, 1, A, n).reshape(n, n).T
    assert np.array_equal(g2[:, 3], Am[:, 3])          # both entries zero: skipped
    assert not np.array_equal(g2[:, 0], Am[:, 0])      # x[0] = 0, y[0] != 0: taken
