"""Pins the oracle's sger / dger restatement (oracle/oracle.c, orc_sger_ld):
the reference's edge cases (tests/{sger,dger}/edge-cases*.json, both layouts)
against numpy and hand values, random strided cases with lda padding,
reference BLAS's quick returns (m or n zero, alpha = 0 reading neither
vector), the skipping of columns whose y entry is zero (Infinity / NaN in x
never meets it; zeros in x are not skipped), and planted mistakes (no
skipping, skipping on x, the transposed update) that these checks reject
(tests/sger/src/test.sger.js:141-298)."""
import numpy as np
import pytest

from oracle import orc
from tests import refcases as rc


def close(a, b, rel=1e-13):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    same = (a == b) | (np.isnan(a) & np.isnan(b))
    scale = np.maximum(np.abs(b), 1.0)
    return bool(np.all(same | (np.abs(a - b) <= rel * scale)))


@pytest.mark.parametrize("routine", ["sger", "dger"])
@pytest.mark.parametrize("cm", [False, True])
def test_edge_cases_against_numpy(routine, cm):
    for c in rc.load(routine, cm):
        call = rc.ger_call(c, np.float64)
        assert np.array_equal(orc.sger_ld(*call), rc.numpy_ger(*call)), c["label"]


def test_hand_values():
    # rectangular 2 x 3 (row-major x = [1, 2], y = [1, 0, -1], A = 0):
    # x y^T = [[1, 0, -1], [2, 0, -2]]
    c = [c for c in rc.load("sger") if c["label"].startswith("rectangular")][0]
    got = orc.sger_ld(*rc.ger_call(c, np.float64))
    assert list(got[:6]) == [1.0, 0.0, -1.0, 2.0, 0.0, -2.0]
    # alpha = -1 subtracts: 10 - 1 * [1, 2]^T [1, 1]
    c = [c for c in rc.load("sger") if c["label"].startswith("alpha=-1")][0]
    assert list(orc.sger_ld(*rc.ger_call(c, np.float64))) == [9.0, 9.0, 8.0, 8.0]


@pytest.mark.parametrize("m,n,inc,pad", [(70, 600, 1, 3), (70, 600, 3, 3), (1100, 150, 8, 0), (1, 1, 2, 5)])
def test_random_strided(m, n, inc, pad):
    lda = m + pad
    x = orc.random_f64((m - 1) * inc + 1, -1, 1, 201)
    y = orc.random_f64((n - 1) * inc + 1, -1, 1, 202)
    A = orc.random_f64(n * lda, -1, 1, 203)
    call = (m, n, 1.5, x, inc, y, inc, A, lda)
    got = orc.sger_ld(*call)
    assert close(got, rc.numpy_ger(*call))
    keep = np.ones(len(A), bool)
    for j in range(n):
        keep[j * lda: j * lda + m] = False
    assert np.array_equal(got[keep], A[keep])  # lda padding untouched


def test_quick_returns_read_neither_vector():
    A = orc.random_f64(16, -1, 1, 9101)
    nan = np.full(4, np.nan)
    for m, n, alpha in ((0, 4, 1.5), (4, 0, 1.5), (4, 4, 0.0)):
        assert np.array_equal(orc.sger_ld(m, n, alpha, nan, 1, nan, 1, A, 4), A)


def test_zero_y_skips_its_column_zero_x_does_not():
    n = 7
    x = orc.random_f64(n, -1, 1, 1)
    y = orc.random_f64(n, -1, 1, 2)
    x[[0, 3]] = 0.0
    y[[1, 3]] = 0.0
    x[1], x[6] = np.inf, -np.inf
    y[5] = np.nan
    A = orc.random_f64(n * n, -1, 1, 3)
    got = orc.sger_ld(n, n, 1.5, x, 1, y, 1, A, n).reshape(n, n).T  # [i, j]
    Am = A.reshape(n, n).T
    assert np.array_equal(got[:, 1], Am[:, 1]) and np.array_equal(got[:, 3], Am[:, 3])
    assert np.all(np.isnan(got[:, 5]))                 # NaN in y: the whole column
    assert np.isinf(got[1, 0]) and np.isinf(got[6, 2])  # Inf in x where y is nonzero
    assert got[0, 0] == Am[0, 0]                        # 0 * (alpha y) adds zero
    # planted mistakes: no skipping (Inf * 0 = NaN in column 1), skipping on x
    with np.errstate(invalid="ignore"):
        no_skip = Am + 1.5 * np.outer(x, y)
    assert np.isnan(no_skip[1, 1]) and not np.isnan(got[1, 1])
    assert np.isnan(got[0, 5])  # x[0] = 0 is not skipped: 0 * NaN (a skip on x would keep it)


def test_transposed_update_rejected():
    m, n = 3, 5
    x = orc.random_f64(m, -1, 1, 4)
    y = orc.random_f64(n, -1, 1, 5)
    A = np.zeros(m * n)
    got = orc.sger_ld(m, n, 2.0, x, 1, y, 1, A, m).reshape(n, m).T
    assert np.allclose(got, 2.0 * np.outer(x, y), rtol=1e-15)
    assert not np.allclose(got[:, :m], 2.0 * np.outer(y, x)[:m, :m])
