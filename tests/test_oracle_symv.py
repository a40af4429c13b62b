"""Pins the oracle's ssymv / dsymv restatement (oracle/oracle.c,
orc_ssymv_ld): the reference's edge cases (tests/{ssymv,dsymv}/edge-cases*.json,
both layouts) against numpy and hand values, random strided cases in both
triangles with the unstored triangle holding NaN (never read), the quick
returns and alpha = 0 rules (tests/ssymv/src/test.ssymv.js:147-171,
258-297), and planted mistakes (the unstored triangle read, the diagonal
counted twice) that these checks reject."""
import numpy as np
import pytest

from oracle import orc
from tests import refcases as rc


def close(a, b, rel=1e-12):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return bool(np.all((a == b) | (np.abs(a - b) <= rel * np.maximum(np.abs(b), 1.0))))


@pytest.mark.parametrize("routine", ["ssymv", "dsymv"])
@pytest.mark.parametrize("cm", [False, True])
def test_edge_cases_against_numpy(routine, cm):
    for c in rc.load(routine, cm):
        call = rc.symv_call(c, np.float64)
        out, _ = orc.ssymv_ld(*call)
        assert np.array_equal(out, rc.numpy_symv(*call)), c["label"]


def test_hand_values():
    # [[1, 2], [2, 3]] [1, 1] = [3, 5] from either stored triangle (99 unread)
    for label in ("lower:", "upper:"):
        c = [c for c in rc.load("ssymv") if c["label"].startswith(label)][0]
        out, _ = orc.ssymv_ld(*rc.symv_call(c, np.float64))
        assert list(out[:2]) == [3.0, 5.0]


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("n,inc,beta", [(70, 1, 0.5), (150, 3, 0.0), (1, 2, 2.0)])
def test_random_strided_unstored_nan(uplo, n, inc, beta):
    lda = n + 2
    A = orc.random_f64(n * lda, -1, 1, 41)
    i, j = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
    unstored = (i < j) if uplo == 1 else (i > j)
    A[(i + j * lda)[unstored]] = np.nan
    x = orc.random_f64((n - 1) * inc + 1, -1, 1, 42)
    y = orc.random_f64((n - 1) * inc + 1, -1, 1, 43)
    call = (uplo, n, 1.5, A, lda, x, inc, beta, y, inc)
    out, ad = orc.ssymv_ld(*call)
    assert np.all(np.isfinite(out)) and close(out, rc.numpy_symv(*call))
    gaps = np.ones(len(y), bool)
    gaps[np.arange(n) * inc] = False
    assert np.array_equal(out[gaps], y[gaps])
    if n > 1:
        # planted: the diagonal counted twice (lower + its transpose, unmasked)
        Ad = np.nan_to_num(rc.dense_op(A, n, n, lda, 0))
        S2 = np.tril(Ad) + np.tril(Ad).T if uplo == 1 else np.triu(Ad) + np.triu(Ad).T
        xv = x[np.arange(n) * inc]
        wrong = 1.5 * (S2 @ xv) + (beta * y[np.arange(n) * inc] if beta else 0)
        assert not close(out[np.arange(n) * inc], wrong)


def test_quick_returns_and_alpha_zero():
    n = 6
    A = orc.random_f64(n * n, -1, 1, 1)
    A[3] = np.nan
    x = np.full(n, np.inf)
    y = orc.random_f64(n, -1, 1, 3)
    out, _ = orc.ssymv_ld(1, n, 0.0, A, n, x, 1, 1.0, y, 1)
    assert np.array_equal(out, y)
    out, _ = orc.ssymv_ld(1, n, 0.0, A, n, x, 1, 0.5, y, 1)
    assert np.array_equal(out, 0.5 * y)
    y0 = y.copy()
    y0[0] = np.nan
    out, _ = orc.ssymv_ld(2, n, 0.0, A, n, x, 1, 0.0, y0, 1)
    assert np.array_equal(out, np.zeros(n))
    out, _ = orc.ssymv_ld(1, 0, 1.5, A, n, x, 1, 0.5, y, 1)
    assert np.array_equal(out, y)
