"""Loads the reference's edge-case fixtures (tests/golden/edge_cases/, copied
data from wgblas's tests/<routine>/edge-cases*.json) and maps each case onto
the column-major C ABI frame, plus an independent numpy expectation.

Layout mapping (the same rule wgblas applies in src/sgemm/sgemm.mjs:151-167,
seen from the column-major side): a row-major m x n matrix with leading
dimension ld is the column-major n x m matrix with the same ld, so a
row-major C = op(A)op(B) is the column-major C^T = op(B)^T op(A)^T: swap A
and B (with their trans flags and ld) and m and n, and flip uplo.
"""
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

TRANS = {"no-transpose": 0, "transpose": 1}
UPLO = {"lower": 1, "upper": 2}


def load(routine, column_major=False):
    suffix = "edge-cases-column-major" if column_major else "edge-cases"
    with open(os.path.join(GOLDEN, "edge_cases", f"{routine}.{suffix}.json")) as f:
        return json.load(f)


def flip_uplo(u):
    return {0: 0, 1: 2, 2: 1}[u]


def gemm_call(case, dtype=np.float32):
    """Column-major call tuple for an sgemm/dgemm/sgemmtr case:
    (uplo, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc)."""
    layout = case.get("layout", "row-major")
    uplo = UPLO.get(case.get("uplo"), 0)
    ta, tb = TRANS[case["transA"]], TRANS[case["transB"]]
    A = np.array(case["A"], dtype)
    B = np.array(case["B"], dtype)
    C = np.array(case["C"], dtype)
    m, n, k = case["m"], case["n"], case["k"]
    lda, ldb, ldc = case["lda"], case["ldb"], case["ldc"]
    if layout == "column-major":
        return (uplo, ta, tb, m, n, k, case["alpha"], A, lda, B, ldb, case["beta"], C, ldc)
    return (flip_uplo(uplo), tb, ta, n, m, k, case["alpha"], B, ldb, A, lda, case["beta"], C, ldc)


def syrk_call(case, dtype=np.float32):
    """Column-major (uplo, trans, n, k, alpha, A, lda, beta, C, ldc) for ssyrk."""
    layout = case.get("layout", "row-major")
    uplo = UPLO[case["uplo"]]
    trans = TRANS[case["trans"]]
    A = np.array(case["A"], dtype)
    C = np.array(case["C"], dtype)
    if layout == "column-major":
        return (uplo, trans, case["n"], case["k"], case["alpha"], A, case["lda"], case["beta"], C,
                case["ldc"])
    return (flip_uplo(uplo), 1 - trans, case["n"], case["k"], case["alpha"], A, case["lda"],
            case["beta"], C, case["ldc"])


def dense_op(buf, rows, cols, ld, trans):
    """op(M) as a dense rows x cols float64 array from a column-major buffer."""
    buf = np.asarray(buf, np.float64)
    i = np.arange(rows)[:, None]
    j = np.arange(cols)[None, :]
    idx = (j + i * ld) if trans else (i + j * ld)
    return buf[idx] if rows and cols else np.zeros((rows, cols))


def numpy_gemm(uplo, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc):
    """Expected column-major C buffer via numpy.matmul (exact for the
    integer-valued fixtures); elements outside m x n / the triangle keep C."""
    out = np.array(C, np.float64, copy=True)
    opA = dense_op(A, m, k, lda, ta)
    opB = dense_op(B, k, n, ldb, tb)
    prod = np.matmul(opA, opB) if alpha != 0 else np.zeros((m, n))
    cij = dense_op(C, m, n, ldc, 0)
    res = alpha * prod + (beta * cij if beta != 0 else 0.0)
    i = np.arange(m)[:, None]
    j = np.arange(n)[None, :]
    mask = np.ones((m, n), bool) if uplo == 0 else ((i >= j) if uplo == 1 else (i <= j))
    idx = (i + j * ldc)[mask]
    out[idx] = res[mask]
    return out


SIDE = {"left": 1, "right": 2}
DIAG = {"non-unit": 0, "unit": 1}


def syr2k_call(case, dtype=np.float32):
    """Column-major (uplo, trans, n, k, alpha, A, lda, B, ldb, beta, C, ldc)
    for ssyr2k: a row-major operand read column-major is its transpose
    (trans flips); the result is symmetric, so a row-major C is the other
    triangle."""
    layout = case.get("layout", "row-major")
    uplo, trans = UPLO[case["uplo"]], TRANS[case["trans"]]
    A, B, C = (np.array(case[x], dtype) for x in "ABC")
    if layout != "column-major":
        uplo, trans = flip_uplo(uplo), 1 - trans
    return (uplo, trans, case["n"], case["k"], case["alpha"], A, case["lda"], B, case["ldb"],
            case["beta"], C, case["ldc"])


def symm_call(case, dtype=np.float32):
    """Column-major (side, uplo, m, n, alpha, A, lda, B, ldb, beta, C, ldc)
    for ssymm: row-major C = S B is column-major C^T = B^T S (side flips, m
    and n swap) and A read column-major stores the other triangle."""
    layout = case.get("layout", "row-major")
    side, uplo = SIDE[case["side"]], UPLO[case["uplo"]]
    m, n = case["m"], case["n"]
    A, B, C = (np.array(case[x], dtype) for x in "ABC")
    if layout != "column-major":
        side, uplo, m, n = 3 - side, flip_uplo(uplo), n, m
    return (side, uplo, m, n, case["alpha"], A, case["lda"], B, case["ldb"], case["beta"], C,
            case["ldc"])


def tri_call(case, dtype=np.float32):
    """Column-major (side, uplo, trans, unit, m, n, alpha, A, lda, B, ldb) for
    strmm / strsm: row-major B = op(A) B is column-major B^T = B^T op(A)^T;
    A read column-major is A^T, so side and uplo flip while trans stays."""
    layout = case.get("layout", "row-major")
    side, uplo = SIDE[case["side"]], UPLO[case["uplo"]]
    trans, unit = TRANS[case["transA"]], DIAG[case["diag"]]
    m, n = case["m"], case["n"]
    A, B = np.array(case["A"], dtype), np.array(case["B"], dtype)
    if layout != "column-major":
        side, uplo, m, n = 3 - side, flip_uplo(uplo), n, m
    return (side, uplo, trans, unit, m, n, case["alpha"], A, case["lda"], B, case["ldb"])


def put(out, vals, ld):
    """Writes the dense rows x cols `vals` into the column-major buffer out."""
    rows, cols = vals.shape
    i = np.arange(rows)[:, None]
    j = np.arange(cols)[None, :]
    out[(i + j * ld).ravel()] = vals.ravel()
    return out


def numpy_syr2k(uplo, trans, n, k, alpha, A, lda, B, ldb, beta, C, ldc):
    opA = dense_op(A, n, k, lda, trans)
    opB = dense_op(B, n, k, ldb, trans)
    prod = opA @ opB.T + opB @ opA.T if alpha != 0 else np.zeros((n, n))
    cij = dense_op(C, n, n, ldc, 0)
    res = alpha * prod + (beta * cij if beta != 0 else 0.0)
    out = np.array(C, np.float64, copy=True)
    i = np.arange(n)[:, None]
    j = np.arange(n)[None, :]
    mask = (i >= j) if uplo == 1 else (i <= j)
    out[(i + j * ldc)[mask]] = res[mask]
    return out


def dense_sym(A, order, lda, uplo):
    """The symmetric matrix whose uplo triangle A stores."""
    full = dense_op(A, order, order, lda, 0)
    tri = np.tril(full) if uplo == 1 else np.triu(full)
    return tri + tri.T - np.diag(np.diag(full))


def dense_tri(A, order, lda, uplo, trans, unit):
    """op(A) of a triangular A: its uplo triangle, zeros elsewhere, unit
    diagonal when unit."""
    full = dense_op(A, order, order, lda, 0)
    tri = np.tril(full) if uplo == 1 else np.triu(full)
    if unit:
        np.fill_diagonal(tri, 1.0)
    return tri.T if trans else tri


def numpy_symm(side, uplo, m, n, alpha, A, lda, B, ldb, beta, C, ldc):
    order = m if side == 1 else n
    S = dense_sym(A, order, lda, uplo)
    Bd = dense_op(B, m, n, ldb, 0)
    prod = (S @ Bd if side == 1 else Bd @ S) if alpha != 0 else np.zeros((m, n))
    res = alpha * prod + (beta * dense_op(C, m, n, ldc, 0) if beta != 0 else 0.0)
    return put(np.array(C, np.float64, copy=True), res, ldc)


def numpy_trmm(side, uplo, trans, unit, m, n, alpha, A, lda, B, ldb):
    order = m if side == 1 else n
    T = dense_tri(A, order, lda, uplo, trans, unit)
    Bd = dense_op(B, m, n, ldb, 0)
    res = alpha * (T @ Bd if side == 1 else Bd @ T) if alpha != 0 else np.zeros((m, n))
    return put(np.array(B, np.float64, copy=True), res, ldb)


def scipy_trsm(side, uplo, trans, unit, m, n, alpha, A, lda, B, ldb):
    """X of op(A) X = alpha B / X op(A) = alpha B by scipy.linalg.solve_triangular."""
    from scipy.linalg import solve_triangular

    order = m if side == 1 else n
    full = dense_op(A, order, order, lda, 0)
    Bd = alpha * dense_op(B, m, n, ldb, 0)
    if alpha == 0:
        X = np.zeros((m, n))
    elif side == 1:
        X = solve_triangular(full, Bd, trans=trans, lower=uplo == 1, unit_diagonal=bool(unit))
    else:
        # X op(A) = B  <=>  op(A)^T X^T = B^T
        X = solve_triangular(full, Bd.T, trans=1 - trans, lower=uplo == 1,
                             unit_diagonal=bool(unit)).T
    return put(np.array(B, np.float64, copy=True), X, ldb)


def gemv_call(case, dtype=np.float32):
    """Column-major (trans, m, n, alpha, A, lda, x, incx, beta, y, incy) for
    sgemv. wgblas's frame is row-major (src/sgemv/sgemv.mjs:97-101): a
    column-major case is first turned into it (m and n swap, trans flips),
    and the row-major mr x nr matrix read column-major is its nr x mr
    transpose (trans flips back)."""
    layout = case.get("layout", "row-major")
    m, n, t = case["m"], case["n"], TRANS[case["trans"]]
    if layout == "column-major":
        m, n, t = n, m, 1 - t
    A, x, y = (np.array(case[k], dtype) for k in ("A", "x", "y"))
    return (1 - t, n, m, case["alpha"], A, case["lda"], x, case["incx"], case["beta"], y, case["incy"])


def ger_call(case, dtype=np.float32):
    """Column-major (m, n, alpha, x, incx, y, incy, A, lda) for sger / dger.
    A row-major m x n A read column-major is A^T (n x m), and the transpose
    of a rank-1 update swaps its vectors (src/sger/sger.mjs:56-64)."""
    layout = case.get("layout", "row-major")
    m, n = case["m"], case["n"]
    x, y, A = (np.array(case[k], dtype) for k in ("x", "y", "A"))
    if layout == "column-major":
        return (m, n, case["alpha"], x, case["incx"], y, case["incy"], A, case["lda"])
    return (n, m, case["alpha"], y, case["incy"], x, case["incx"], A, case["lda"])


def numpy_ger(m, n, alpha, x, incx, y, incy, A, lda):
    """Column-major A + alpha x y^T by numpy (float64), with reference BLAS's
    quick returns and its skipping of columns whose y entry is zero."""
    out = np.array(A, np.float64, copy=True)
    if m == 0 or n == 0 or alpha == 0:
        return out
    xv = np.asarray(x, np.float64)[np.arange(m) * incx]
    yv = np.asarray(y, np.float64)[np.arange(n) * incy]
    for j in np.nonzero(yv != 0)[0]:
        col = out[j * lda: j * lda + m]
        col += xv * (alpha * yv[j])
    return out


def syr_call(case, dtype=np.float32):
    """Column-major (uplo, n, alpha, x, incx, A, lda) for ssyr / dsyr, or
    (uplo, n, alpha, x, incx, y, incy, A, lda) for ssyr2 / dsyr2 (a case with
    y). A symmetric row-major A read column-major stores the other triangle:
    uplo flips (src/ssyr/ssyr.mjs:68-71)."""
    uplo = UPLO[case["uplo"]]
    if case.get("layout", "row-major") != "column-major":
        uplo = flip_uplo(uplo)
    x, A = np.array(case["x"], dtype), np.array(case["A"], dtype)
    if "y" in case:
        return (uplo, case["n"], case["alpha"], x, case["incx"], np.array(case["y"], dtype), case["incy"],
                A, case["lda"])
    return (uplo, case["n"], case["alpha"], x, case["incx"], A, case["lda"])


def numpy_syr2(uplo, n, alpha, x, incx, y, incy, A, lda):
    """Column-major ssyr2 (y given) / ssyr (y None) by numpy (float64): the
    uplo triangle of A + alpha (x y^T + y x^T) (or + alpha x x^T), with the
    quick returns and the skip of columns whose x (and y) entry is zero."""
    out = np.array(A, np.float64, copy=True)
    if n == 0 or alpha == 0:
        return out
    xv = np.asarray(x, np.float64)[np.arange(n) * incx]
    yv = xv if y is None else np.asarray(y, np.float64)[np.arange(n) * incy]
    for j in range(n):
        if xv[j] == 0 and (y is None or yv[j] == 0):
            continue
        rows = np.arange(j, n) if uplo == 1 else np.arange(0, j + 1)
        upd = xv[rows] * (alpha * yv[j])
        if y is not None:
            upd = upd + yv[rows] * (alpha * xv[j])
        out[rows + j * lda] += upd
    return out


def symv_call(case, dtype=np.float32):
    """Column-major (uplo, n, alpha, A, lda, x, incx, beta, y, incy) for
    ssymv / dsymv: a symmetric row-major A read column-major stores the
    other triangle, so uplo flips (src/ssymv/ssymv.mjs:96-99)."""
    uplo = UPLO[case["uplo"]]
    if case.get("layout", "row-major") != "column-major":
        uplo = flip_uplo(uplo)
    A, x, y = (np.array(case[k], dtype) for k in ("A", "x", "y"))
    return (uplo, case["n"], case["alpha"], A, case["lda"], x, case["incx"], case["beta"], y, case["incy"])


def numpy_symv(uplo, n, alpha, A, lda, x, incx, beta, y, incy):
    """Column-major symv by numpy (float64): S from A's uplo triangle, with
    reference BLAS's quick returns."""
    out = np.array(y, np.float64, copy=True)
    if n == 0 or (alpha == 0 and beta == 1):
        return out
    Ad = dense_op(A, n, n, lda, 0)
    S = np.tril(Ad) + np.tril(Ad, -1).T if uplo == 1 else np.triu(Ad) + np.triu(Ad, 1).T
    xv = np.asarray(x, np.float64)[np.arange(n) * incx]
    prod = S @ xv if alpha != 0 else np.zeros(n)
    idx = np.arange(n) * incy
    yin = out[idx]
    out[idx] = alpha * prod + (beta * yin if beta != 0 else 0.0)
    return out


def numpy_gemv(trans, m, n, alpha, A, lda, x, incx, beta, y, incy):
    """Column-major sgemv by numpy (float64), with reference BLAS's quick
    returns and the no-transpose form's skipping of zero x entries."""
    out = np.array(y, np.float64, copy=True)
    if m == 0 or n == 0 or (alpha == 0 and beta == 1):
        return out
    Ad = dense_op(A, m, n, lda, 0)
    xl = n if trans == 0 else m
    xv = np.asarray(x, np.float64)[np.arange(xl) * incx]
    if alpha == 0:
        prod = np.zeros(m if trans == 0 else n)
    elif trans == 0:
        keep = xv != 0
        prod = Ad[:, keep] @ xv[keep]
    else:
        prod = Ad.T @ xv
    idx = np.arange(len(prod)) * incy
    yin = out[idx]
    out[idx] = alpha * prod + (beta * yin if beta != 0 else 0.0)
    return out


def trmv_call(case, dtype=np.float32):
    """Column-major (uplo, trans, diag, n, A, lda, x, incx, y, incy) for
    strmv / dtrmv: a row-major A read column-major is A^T, so uplo and trans
    both flip (src/strmv/strmv.mjs:97-103). y is output only; it is sized
    from n and incy where the case holds none."""
    uplo, trans = UPLO[case["uplo"]], TRANS[case["trans"]]
    if case.get("layout", "row-major") != "column-major":
        uplo, trans = flip_uplo(uplo), 1 - trans
    A, x = (np.array(case[k], dtype) for k in ("A", "x"))
    n, incy = case["n"], case["incy"]
    y = np.array(case["y"], dtype) if "y" in case else np.zeros(max(n - 1, 0) * incy + 1, dtype)
    return (uplo, trans, DIAG[case["diag"]], n, A, case["lda"], x, case["incx"], y, incy)


def numpy_trmv(uplo, trans, diag, n, A, lda, x, incx, y, incy):
    """Column-major strmv by numpy (float64): op(T) x into y's strided slots,
    T the uplo triangle of A (unit diagonal 1); the no-transpose column form
    drops the columns where x is zero."""
    out = np.array(y, np.float64, copy=True)
    if n == 0:
        return out
    Ad = dense_op(A, n, n, lda, 0)
    T = np.tril(Ad) if uplo == 1 else np.triu(Ad)
    if diag == 1:
        np.fill_diagonal(T, 1.0)
    xv = np.asarray(x, np.float64)[np.arange(n) * incx]
    if trans == 0:
        keep = xv != 0
        out[np.arange(n) * incy] = T[:, keep] @ xv[keep]
    else:
        out[np.arange(n) * incy] = T.T @ xv
    return out
