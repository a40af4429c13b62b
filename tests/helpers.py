"""Shared checks for the parity tests.

The error metrics restate the reference's own test bounds:
  * GEMM forward factor (tests/sgemm/helpers.js:1-57, restricted to the
    triangle for sgemmtr/ssyrk as in tests/sgemmtr/helpers.js):
        |C - C_ref| <= eps*((k+1)|alpha| sum_p |a b| + |beta||C_in|), eps = 2^-23
  * dgemm (tests/dgemm/helpers.js:1-63): eps = 2^-48 with (k+2) and 3|beta||C_in|
  * sdot (tests/sdot/helpers.js): |dot - ref| <= n*eps*sum|x y|
  * sasum / snrm2: <= 50 ULP (tests/sasum/src/test.sasum.js:43,
    tests/snrm2/src/test.snrm2.js:43), ULP as tests/helpers/ulp.js (+-0 equal)
  * isamax: exact index.
Here C_ref is the oracle's long-double result, which is at least as strict as
the reference's comparison against stdlib's float32 result.
"""
import numpy as np

EPS32 = 2.0 ** -23
EPS_DD = 2.0 ** -48


def ulp_diff32(a, b):
    """tests/helpers/ulp.js ulpDiff: bit distance of two float32s, +-0 equal."""
    a = np.float32(a)
    b = np.float32(b)
    if a == 0 and b == 0:
        return 0
    ia = int(np.array(a, np.float32).view(np.uint32))
    ib = int(np.array(b, np.float32).view(np.uint32))
    return abs(ia - ib)


def col_major_elems(rows, cols, ld):
    """Length of a column-major rows x cols matrix with leading dimension ld
    stored as cols full columns (padding included), as GpuMatrix stores it."""
    return max(cols, 1) * ld


def gemm_forward_factor(got, ref, absdot, cin, m, n, k, alpha, beta, ldc, uplo=0, dd=False):
    """Max over the (uplo part of the) m x n C of |got-ref| / bound."""
    got = np.asarray(got, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    j = np.arange(n)[None, :]
    i = np.arange(m)[:, None]
    idx = (i + j * ldc).reshape(-1)
    mask = np.ones((m, n), bool)
    if uplo == 1:
        mask = i >= j
    elif uplo == 2:
        mask = i <= j
    mask = mask.reshape(-1)
    idx = idx[mask]
    g, r = got[idx], ref[idx]
    a = np.asarray(absdot, np.float64).reshape(-1)[idx]
    c = np.abs(np.asarray(cin, np.float64).reshape(-1)[idx])
    if dd:
        bound = EPS_DD * ((k + 2) * abs(alpha) * a + 3 * abs(beta) * c)
    else:
        bound = EPS32 * ((k + 1) * abs(alpha) * a + abs(beta) * c)
    err = np.abs(g - r)
    with np.errstate(invalid="ignore", divide="ignore"):
        fac = np.where(bound == 0, np.where(err == 0, 0.0, np.inf), err / np.where(bound == 0, 1, bound))
    return float(fac.max()) if fac.size else 0.0


def untouched_mask(m, n, ldc, ncols, uplo=0):
    """Boolean mask over a (ldc*ncols) column-major buffer: True where the
    routine must leave C bit-identical (ld padding, other triangle)."""
    total = ldc * ncols
    keep = np.ones(total, bool)
    j = np.arange(n)[None, :]
    i = np.arange(m)[:, None]
    inside = np.ones((m, n), bool)
    if uplo == 1:
        inside = i >= j
    elif uplo == 2:
        inside = i <= j
    idx = (i + j * ldc)[inside]
    keep[idx] = False
    return keep


def bits_equal(a, b):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    if a.dtype == np.float32:
        return np.array_equal(a.view(np.uint32), b.view(np.uint32))
    return np.array_equal(a.view(np.uint64), b.view(np.uint64))


def cm_view(flat, rows, cols, ld):
    """Column-major (rows x cols, leading dimension ld) view of a flat array."""
    need = cols * ld
    buf = flat if flat.size >= need else np.concatenate([flat, np.zeros(need - flat.size, flat.dtype)])
    return buf[:need].reshape(cols, ld).T[:rows, :]


def op(M, trans):
    return M.T if trans else M


def check_gemm_props(C, C0, opA, opB, alpha, beta, k, eps=EPS32, kterm=1, cterm=1.0, rows=(),
                     cols=(), seed=0, uplo=0):
    """C, C0: m x n views; opA m x k; opB k x n (any float dtype)."""
    m, n = C.shape
    rng = np.random.default_rng(seed)
    A64 = np.asarray(opA, np.float64)
    B64 = np.asarray(opB, np.float64)
    rows = sorted(set([0, 1, m - 1] + list(rows) + [int(r) for r in rng.integers(0, m, 8)]))
    cols = sorted(set([0, 1, n - 1] + list(cols) + [int(c) for c in rng.integers(0, n, 8)]))
    worst = 0.0
    for sel_r, sel_c in ((rows, slice(None)), (slice(None), cols)):
        exact = alpha * (A64[sel_r, :] @ B64[:, sel_c]) + beta * np.asarray(C0[sel_r, sel_c], np.float64)
        absd = np.abs(A64[sel_r, :]) @ np.abs(B64[:, sel_c])
        bound = eps * ((k + kterm) * abs(alpha) * absd + cterm * abs(beta) * np.abs(np.asarray(C0[sel_r, sel_c], np.float64)))
        got = np.asarray(C[sel_r, sel_c], np.float64)
        if uplo:
            i = np.arange(m)[sel_r][:, None] if not isinstance(sel_r, slice) else np.arange(m)[:, None]
            j = np.arange(n)[sel_c][None, :] if not isinstance(sel_c, slice) else np.arange(n)[None, :]
            mask = (i >= j) if uplo == 1 else (i <= j)
            err = np.where(mask, np.abs(got - exact), 0.0)
        else:
            err = np.abs(got - exact)
        assert np.all(err <= bound), f"forward factor {np.max(err / np.where(bound > 0, bound, 1))}"
        worst = max(worst, float(np.max(err / np.where(bound > 0, bound, np.inf))))
    if uplo == 0:
        for t in range(2):
            x = rng.choice([-1.0, 1.0], size=n)
            lhs = np.asarray(C, np.float64) @ x
            rhs = alpha * (A64 @ (B64 @ x)) + beta * (np.asarray(C0, np.float64) @ x)
            tol = eps * ((k + kterm) * abs(alpha) * (np.abs(A64) @ (np.abs(B64) @ np.abs(x)))
                         + cterm * abs(beta) * (np.abs(np.asarray(C0, np.float64)) @ np.abs(x)))
            tol += 1e-12 * (np.abs(lhs) + np.abs(rhs))
            assert np.all(np.abs(lhs - rhs) <= tol), "Freivalds projection exceeds the summed bound"
    return worst
