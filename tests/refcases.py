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
