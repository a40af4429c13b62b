"""Pins the oracle's ssyr2k / ssymm / strmm / strsm restatements
(oracle/oracle.c, orc_*_ld; dsyr2k / dsymm / dtrmm use the first three on
doubles) before the GPU tests trust them.

Checks: every reference edge case (tests/<routine>/edge-cases*.json, both
layouts) against an independent numpy product (or scipy's
solve_triangular), random cases over every side / uplo / trans / diag with
ld padding, the alpha = 0 rules of the reference's "reads neither A nor B"
regressions, and planted mistakes (a dropped term, a wrong triangle, a
transposed operand) that these checks must reject.
"""
import itertools

import numpy as np
import pytest

from oracle import orc
from tests import refcases as rc


def close(a, b, rel=1e-12):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    scale = max(1.0, float(np.max(np.abs(b))) if b.size else 1.0)
    return bool(np.all((a == b) | (np.abs(a - b) <= rel * scale)))


# ------------------------------------------------------------ edge cases
# the fp64 routines (dsyr2k / dsymm / dtrmm) run the same restatements on
# doubles: their own fixtures pin them too
@pytest.mark.parametrize("routine", ["ssyr2k", "dsyr2k"])
@pytest.mark.parametrize("cm", [False, True])
def test_syr2k_edge_cases(routine, cm):
    for c in rc.load(routine, cm):
        call = rc.syr2k_call(c, np.float64)
        out, _, _ = orc.ssyr2k_ld(*call)
        assert close(out, rc.numpy_syr2k(*call)), c["label"]


@pytest.mark.parametrize("routine", ["ssymm", "dsymm"])
@pytest.mark.parametrize("cm", [False, True])
def test_symm_edge_cases(routine, cm):
    for c in rc.load(routine, cm):
        call = rc.symm_call(c, np.float64)
        out, _ = orc.ssymm_ld(*call)
        assert close(out, rc.numpy_symm(*call)), c["label"]


@pytest.mark.parametrize("routine", ["strmm", "dtrmm"])
@pytest.mark.parametrize("cm", [False, True])
def test_trmm_edge_cases(routine, cm):
    for c in rc.load(routine, cm):
        call = rc.tri_call(c, np.float64)
        out, _ = orc.strmm_ld(*call)
        assert close(out, rc.numpy_trmm(*call)), c["label"]


@pytest.mark.parametrize("cm", [False, True])
def test_strsm_edge_cases(cm):
    for c in rc.load("strsm", cm):
        call = rc.tri_call(c, np.float64)
        assert close(orc.strsm_ld(*call), rc.scipy_trsm(*call), 1e-12), c["label"]


def test_edge_case_hand_values():
    # ssyr2k lower, A = [[1,2],[3,4]], B = [[5,6],[7,8]] row-major, alpha 1:
    # A B^T = [[17, 23], [39, 53]], so A B^T + B A^T = [[34, 62], [62, 106]]
    c = dict(label="hand", uplo="lower", trans="no-transpose", n=2, k=2, alpha=1,
             A=[1, 2, 3, 4], lda=2, B=[5, 6, 7, 8], ldb=2, beta=0, C=[9, 9, 9, 9], ldc=2)
    out, _, _ = orc.ssyr2k_ld(*rc.syr2k_call(c, np.float64))
    assert list(out) == [34.0, 9.0, 62.0, 106.0]  # row-major [[34, 9], [62, 106]]
    # strsm left lower non-unit, row-major A = [[2,0],[1,4]], B = [[2],[9]]:
    # x0 = 1, x1 = (9 - 1) / 4 = 2
    c = dict(side="left", uplo="lower", transA="no-transpose", diag="non-unit", m=2, n=1,
             alpha=1, A=[2, 0, 1, 4], lda=2, B=[2, 9], ldb=1)
    assert list(orc.strsm_ld(*rc.tri_call(c, np.float64))) == [1.0, 2.0]
    # strmm of the same: B = A x = [2, 9]
    c["B"] = [1, 2]
    out, _ = orc.strmm_ld(*rc.tri_call(c, np.float64))
    assert list(out) == [2.0, 9.0]


# ------------------------------------------------------------ random cases
def rnd(n, seed):
    return orc.random_f32(n, -1.0, 1.0, seed).astype(np.float64)


@pytest.mark.parametrize("uplo,trans", list(itertools.product([1, 2], [0, 1])))
def test_ssyr2k_random(uplo, trans):
    n, k = 37, 13
    lda = (k if trans else n) + 2
    ldb = (k if trans else n) + 1
    ldc = n + 3
    cols = n if trans else k
    A, B, C = rnd(lda * cols, 1), rnd(ldb * cols, 2), rnd(ldc * n, 3)
    call = (uplo, trans, n, k, 1.5, A, lda, B, ldb, 0.5, C, ldc)
    out, a1, a2 = orc.ssyr2k_ld(*call)
    assert close(out, rc.numpy_syr2k(*call))
    # planted mistake: only the first product -> must differ
    one, _ = orc.gemm_ld(uplo, trans, 1 - trans, n, n, k, 1.5, A, lda, B, ldb, 0.5, C, ldc)
    assert not close(one, out, 1e-6)
    assert np.all(a1 >= 0) and np.all(a2 >= 0)


@pytest.mark.parametrize("side,uplo", list(itertools.product([1, 2], [1, 2])))
def test_ssymm_random(side, uplo):
    m, n = 29, 17
    order = m if side == 1 else n
    lda, ldb, ldc = order + 2, m + 1, m + 3
    A, B, C = rnd(lda * order, 4), rnd(ldb * n, 5), rnd(ldc * n, 6)
    call = (side, uplo, m, n, -0.75, A, lda, B, ldb, 2.0, C, ldc)
    out, _ = orc.ssymm_ld(*call)
    assert close(out, rc.numpy_symm(*call))
    # planted mistake: the other triangle read as the stored one
    assert not close(out, rc.numpy_symm(side, 3 - uplo, *call[2:]), 1e-6)
    # NaN in the unstored triangle is never read
    Anan = A.copy()
    i, j = (0, order - 1) if uplo == 1 else (order - 1, 0)
    Anan[i + j * lda] = np.nan
    out2, _ = orc.ssymm_ld(side, uplo, m, n, -0.75, Anan, lda, B, ldb, 2.0, C, ldc)
    assert np.array_equal(out2, out)


@pytest.mark.parametrize("side,uplo,trans,unit",
                         list(itertools.product([1, 2], [1, 2], [0, 1], [0, 1])))
def test_strmm_strsm_random(side, uplo, trans, unit):
    m, n = 23, 19
    order = m if side == 1 else n
    lda, ldb = order + 1, m + 2
    A = rnd(lda * order, 7) / order
    for d in range(order):
        A[d + d * lda] = 2.0 + 0.25 * (d % 3)
    B = rnd(ldb * n, 8)
    call = (side, uplo, trans, unit, m, n, 1.25, A, lda, B, ldb)
    out, _ = orc.strmm_ld(*call)
    assert close(out, rc.numpy_trmm(*call))
    X = orc.strsm_ld(*call)
    assert close(X, rc.scipy_trsm(*call), 1e-12)
    # round trip: strmm of the solution gives back alpha * B
    back, _ = orc.strmm_ld(side, uplo, trans, unit, m, n, 1.0, A, lda, X, ldb)
    Bd = rc.dense_op(B, m, n, ldb, 0)
    assert np.allclose(rc.dense_op(back, m, n, ldb, 0), 1.25 * Bd, rtol=0, atol=1e-12)
    # ld padding of B untouched
    pad = np.ones(ldb * n, bool)
    pad[(np.arange(m)[:, None] + np.arange(n)[None, :] * ldb).ravel()] = False
    assert np.array_equal(X[pad], B[pad]) and np.array_equal(out[pad], B[pad])
    # planted mistake: the transposed triangle
    assert not close(X, rc.scipy_trsm(side, uplo, 1 - trans, *call[3:]), 1e-6)


def test_alpha_zero_reads_neither_a_nor_b():
    # tests/{ssyr2k,ssymm,strmm}/src/test.*.js "alpha = 0 reads neither A nor B",
    # tests/strsm/src/test.strsm.js "alpha=0 — poisoned B becomes a literal zero"
    n = 7
    A = rnd(n * n, 1)
    A[3 + 1 * n] = np.nan
    B = rnd(n * n, 2)
    B[2 + 3 * n] = np.inf
    B[0] = np.nan
    C = rnd(n * n, 3)
    out, _, _ = orc.ssyr2k_ld(1, 0, n, n, 0.0, A, n, B, n, 0.5, C, n)
    i, j = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
    low = (i >= j).ravel(order="F")
    assert np.array_equal(out[low], 0.5 * C[low]) and np.array_equal(out[~low], C[~low])
    Cn = C.copy()
    Cn[4 + 4 * n] = np.nan
    out, _ = orc.ssymm_ld(1, 1, n, n, 0.0, A, n, B, n, 0.0, Cn, n)
    assert np.array_equal(out, np.zeros(n * n))
    out, _ = orc.strmm_ld(2, 1, 0, 0, n, n, 0.0, A, n, B, n)
    assert np.array_equal(out, np.zeros(n * n))
    assert np.array_equal(orc.strsm_ld(1, 1, 0, 0, n, n, 0.0, A, n, B, n), np.zeros(n * n))


def test_strsm_ieee_specials_follow_substitution():
    # tests/strsm/src/test.strsm.js:524-578: Infinity in B propagates along
    # the solve order; NaN in the unreferenced triangle is never read
    m, n = 7, 5
    A = rnd(m * m, 1)
    for d in range(m):
        A[d + d * m] += m + 4
    A[1 + 4 * m] = np.nan  # row 1, col 4: the upper triangle, unread by a lower solve
    B = rnd(m * n, 2)
    B[1 + 2 * m] = np.inf  # column 2, row 1
    X = orc.strsm_ld(1, 1, 0, 0, m, n, 1.0, A.copy(), m, B, m)
    Xd = rc.dense_op(X, m, n, m, 0)
    assert np.all(np.isfinite(np.delete(Xd, 2, axis=1)))  # other columns finite
    assert np.all(np.isfinite(Xd[:1, 2])) and np.isinf(Xd[1, 2])
    assert np.all(~np.isfinite(Xd[2:, 2]))  # later rows of that column: Inf or NaN
