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
    rows = sorted(r for r in set([0, 1, m - 1] + list(rows) + [int(r) for r in rng.integers(0, m, 8)])
                  if r < m)
    cols = sorted(c for c in set([0, 1, n - 1] + list(cols) + [int(c) for c in rng.integers(0, n, 8)])
                  if c < n)
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


def run_gemm_props_case(ctx, kind, uplo, ta, tb, m, n, k, alpha, beta, ldc_pad=3, seed=11,
                        lda_pad=0, ldb_pad=0):
    """Runs sgemm / sgemmtr / ssyrk / dgemm through the C ABI on device-seeded
    inputs and checks the result with check_gemm_props (sampled rows and
    columns plus a Freivalds projection) and bit checks of what must stay."""
    dt = np.float64 if kind == "dgemm" else np.float32
    a_rows, a_cols = (k, m) if ta else (m, k)
    if kind == "ssyrk":
        tb = 1 - ta
        b_rows, b_cols = a_rows, a_cols
    else:
        b_rows, b_cols = (n, k) if tb else (k, n)
    lda, ldb, ldc = a_rows + lda_pad, b_rows + ldb_pad, m + ldc_pad
    sa, sb, sc = lda * a_cols, ldb * b_cols, ldc * n
    buf = ctx.empty(sa + sb + sc, dt)
    ctx.fill_uniform(buf, -1.0, 1.0, seed)
    host = buf.to_host()
    A, C0 = host[:sa], host[sa + sb:]
    B = A if kind == "ssyrk" else host[sa:sa + sb]
    pa, pb, pc = buf.offset(0), buf.offset(sa), buf.offset(sa + sb)
    if kind == "dgemm":
        ctx.dgemm(ta, tb, m, n, k, alpha, pa, lda, pb, ldb, beta, pc, ldc)
    elif kind == "ssyrk":
        ctx.ssyrk(uplo, ta, n, k, alpha, pa, lda, beta, pc, ldc)
    elif uplo:
        ctx.sgemmtr(uplo, ta, tb, m, n, k, alpha, pa, lda, pb, ldb, beta, pc, ldc)
    else:
        ctx.sgemm(ta, tb, m, n, k, alpha, pa, lda, pb, ldb, beta, pc, ldc)
    C = buf.to_host()[sa + sb:]
    buf.free()
    keep = untouched_mask(m, n, ldc, n, uplo)
    assert bits_equal(C[keep], C0[keep]), "C changed outside its m x n part / triangle"
    Am = op(cm_view(A, a_rows, a_cols, lda), ta)
    Bm = op(cm_view(B, b_rows, b_cols, ldb), tb)
    edges = (0, 63, 64, 127, 128, 255, 256, m - 1, n - 1)
    kw = dict(eps=EPS_DD, kterm=2, cterm=3.0) if kind == "dgemm" else {}
    check_gemm_props(cm_view(C, m, n, ldc), cm_view(C0, m, n, ldc), Am, Bm, alpha, beta, k,
                     rows=tuple(r for r in edges if r < m), cols=tuple(c for c in edges if c < n),
                     seed=seed, uplo=uplo, **kw)
