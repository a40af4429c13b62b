"""GPU parity of sger and dger (rank-1 updates) through the C ABI against
the oracle's long-double restatement, under the reference's metric
(tests/sger/helpers.js, tests/dger/helpers.js): |A - A_ref| <= eps
(|alpha x y| + |A_in|) elementwise, eps = 2^-23 with factor <= 2 for sger (the
reference's THRESHOLD), 2^-48 with factor <= 1 for dger. The edge cases are
held to exact equality and the IEEE regressions to the same NaN / Inf
positions, as the reference's tests do; lda padding must come back
bit-identical. The scenarios follow tests/sger/src/test.sger.js and
tests/dger/src/test.dger.js; dger's "f32 exponent range" regression describes
double-double's range, so its inputs are checked in f64's range instead.
Cases are written in the reference's terms and mapped onto the column-major
C ABI as the JS layer does (tests/refcases.py)."""
import numpy as np
import pytest

from oracle import orc
from tests import refcases as rc
from tests.helpers import EPS32, EPS_DD, bits_equal

pytestmark = pytest.mark.gpu

PREC = {"sger": (np.float32, EPS32, 2.0), "dger": (np.float64, EPS_DD, 1.0)}


def up(ctx, a, dt):
    a = np.asarray(a, dt)
    return ctx.upload(a if a.size else np.zeros(1, dt))


def run(ctx, r, call):
    dt = PREC[r][0]
    m, n, alpha, x, incx, y, incy, A, lda = call
    dA = up(ctx, A, dt)
    getattr(ctx, r)(m, n, alpha, up(ctx, x, dt), incx, up(ctx, y, dt), incy, dA, lda)
    return dA.to_host()[: len(A)]


def region(m, n, lda):
    """Indices of the m x n column-major matrix, (i, j) in row order (j fastest,
    as np.outer(x, y).ravel())."""
    i = np.arange(m)[:, None]
    j = np.arange(n)[None, :]
    return (i + j * lda).ravel()


def check(ctx, r, call, exact=False):
    dt, eps, threshold = PREC[r]
    m, n, alpha, x, incx, y, incy, A, lda = call
    got = run(ctx, r, call)
    ref = orc.sger_ld(*call)
    if exact:
        assert bits_equal(got, ref.astype(dt))
        return got
    idx = region(m, n, lda)
    g, rf = got[idx].astype(np.float64), ref[idx]
    assert np.array_equal(np.isnan(g), np.isnan(rf))
    inf = np.isinf(rf)
    assert np.array_equal(g[inf], rf[inf])
    xv = np.asarray(x, np.float64)[np.arange(m) * incx]
    yv = np.asarray(y, np.float64)[np.arange(n) * incy]
    with np.errstate(invalid="ignore", over="ignore"):
        bound = eps * (np.abs(alpha * np.outer(xv, yv)).ravel() + np.abs(np.asarray(A, np.float64)[idx]))
    fin = np.isfinite(rf)
    err = np.abs(g[fin] - rf[fin])
    assert np.all((err <= threshold * bound[fin]) | (err == 0))
    keep = np.ones(len(A), bool)
    keep[idx] = False
    assert bits_equal(got[keep], np.asarray(A, dt)[keep])  # lda padding untouched
    return got


def at(n, i, j):
    return i * n + j


@pytest.mark.parametrize("r", ["sger", "dger"])
@pytest.mark.parametrize("cm", [False, True])
def test_edge_cases_exact(ctx, r, cm):
    # test.sger.js:105-139, 180-217 (deepEqual against stdlib); dger's the same
    for c in rc.load(r, cm):
        check(ctx, r, rc.ger_call(c, PREC[r][0]), exact=True)


@pytest.mark.parametrize("r", ["sger", "dger"])
def test_zero_dimension_leaves_a(ctx, r):
    # test.sger.js:141-178: m = 0, n = 0 with a realistic lda
    dt = PREC[r][0]
    for m, n in ((0, 4), (4, 0)):
        A = orc.random_f64(16, -1, 1, 9101 + m).astype(dt)
        got = run(ctx, r, (m, n, 1.5, orc.random_f64(4, -1, 1, 9102), 1, orc.random_f64(4, -1, 1, 9103),
                           1, A, 4))
        assert bits_equal(got, A)


@pytest.mark.parametrize("r", ["sger", "dger"])
@pytest.mark.parametrize("layout", ["row-major", "column-major"])
@pytest.mark.parametrize("n", [7, 300])
def test_zero_vector_entries_skip_their_row(ctx, r, layout, n):
    # test.sger.js:219-266: zeros next to Infinity and NaN, stride 2
    dt = PREC[r][0]
    inc = 2
    ln = (n - 1) * inc + 1
    x = orc.random_f64(ln, -1, 1, 1)
    y = orc.random_f64(ln, -1, 1, 2)
    for i in (0, 3, 5):
        x[i * inc] = 0
    for i in (1, 3, 6):
        y[i * inc] = 0
    x[1 * inc], x[6 * inc], y[5 * inc] = np.inf, -np.inf, np.nan
    c = dict(layout=layout, m=n, n=n, alpha=1.5, x=x, incx=inc, y=y, incy=inc,
             A=orc.random_f64(n * n, -1, 1, 3), lda=n)
    got = check(ctx, r, rc.ger_call(c, dt))
    assert np.isnan(got).any() and np.isinf(got).any()


@pytest.mark.parametrize("r", ["sger", "dger"])
def test_alpha_zero_leaves_a(ctx, r):
    # test.sger.js:268-298: x holds Infinity and NaN, never read
    dt = PREC[r][0]
    n = 6
    x = orc.random_f64(n, -1, 1, 1)
    x[1], x[3] = np.inf, np.nan
    A = orc.random_f64(n * n, -1, 1, 3).astype(dt)
    c = dict(m=n, n=n, alpha=0.0, x=x, incx=1, y=orc.random_f64(n, -1, 1, 2), incy=1, A=A, lda=n)
    assert bits_equal(run(ctx, r, rc.ger_call(c, dt)), A)


@pytest.mark.parametrize("r", ["sger", "dger"])
@pytest.mark.parametrize("M,N,inc", [(70, 600, 1), (70, 600, 3), (1100, 150, 8)])
@pytest.mark.parametrize("layout", ["row-major", "column-major"])
def test_multi_chunk_and_strides(ctx, r, M, N, inc, layout):
    # test.dger.js:202-256: lda = inner + 3 (padding checked bit for bit)
    dt = PREC[r][0]
    cm = layout == "column-major"
    inner, outer = (M, N) if cm else (N, M)
    lda = inner + 3
    c = dict(layout=layout, m=M, n=N, alpha=1.5, x=orc.random_f64((M - 1) * inc + 1, -1, 1, 201), incx=inc,
             y=orc.random_f64((N - 1) * inc + 1, -1, 1, 202), incy=inc,
             A=orc.random_f64(outer * lda, -1, 1, 203), lda=lda)
    check(ctx, r, rc.ger_call(c, dt))


def test_dger_exactness_and_ieee(ctx):
    # test.dger.js:295-347: alpha = 0 returns A bit for bit; lda padding;
    # Infinity in x, NaN in y, -Infinity in A propagate as in real f64
    full = lambda size, s: orc.random_f64(size, -1, 1, s) * np.pi  # noqa: E731
    m, n = 4, 5
    A = full(m * n, 1000)
    assert bits_equal(run(ctx, "dger", (n, m, 0.0, full(n, 1), 1, full(m, 2), 1, A, n)), A)
    check(ctx, "dger", rc.ger_call(dict(m=m, n=n, alpha=1.5, x=full(m, 3), incx=1, y=full(n, 4), incy=1,
                                        A=full(m * (n + 3), 5), lda=n + 3), np.float64))
    for n in (7, 300):
        x = orc.random_f64(n, -1, 1, 1)
        x[2] = np.inf
        y = orc.random_f64(n, -1, 1, 2)
        y[3] = np.nan
        A = orc.random_f64(n * n, -1, 1, 3)
        A[at(n, 5, 5)] = -np.inf
        got = check(ctx, "dger", rc.ger_call(dict(m=n, n=n, alpha=1.5, x=x, incx=1, y=y, incy=1, A=A,
                                                  lda=n), np.float64))
        assert np.isnan(got).any() and np.isinf(got).any()


@pytest.mark.parametrize("n", [7, 300])
def test_dger_f64_exponent_range(ctx, n):
    # the inputs of test.dger.js:349-420 in f64's range: 1e300 and 1e-50 read
    # as they are, a product past 3.4e38 stays finite
    x = orc.random_f64(n, -1, 1, 1)
    x[2], x[4] = 1e300, 1e-50
    A = orc.random_f64(n * n, -1, 1, 3)
    A[at(n, 0, n - 1)] = -1e300
    got = check(ctx, "dger", rc.ger_call(dict(m=n, n=n, alpha=1.5, x=x, incx=1,
                                              y=orc.random_f64(n, -1, 1, 2), incy=1, A=A, lda=n),
                                         np.float64))
    assert np.all(np.isfinite(got)) and np.abs(got).max() > 1e299
    x = orc.random_f64(n, -1, 1, 1)
    x[2] = 1e30
    got = check(ctx, "dger", rc.ger_call(dict(m=n, n=n, alpha=1e10, x=x, incx=1,
                                              y=orc.random_f64(n, -1, 1, 2), incy=1,
                                              A=orc.random_f64(n * n, -1, 1, 3), lda=n), np.float64))
    assert np.all(np.isfinite(got)) and np.abs(got).max() > 3.4e38


@pytest.mark.parametrize("r", ["sger", "dger"])
@pytest.mark.parametrize("shape", [(4096, 4096, 4096), (65536, 48, 65536), (48, 65536, 49),
                                   (3001, 2999, 3003), (1024, 9, 1025)])
def test_large_and_skinny(ctx, r, shape):
    # one row block (48 rows) or one column chunk, odd sizes with odd lda
    # (element loads), x misaligned by one element
    dt = PREC[r][0]
    m, n, lda = shape
    x = orc.random_f64(m + 1, -1, 1, 41)
    call = (m, n, 0.75, x[1:], 1, orc.random_f64(n, -1, 1, 42), 1, orc.random_f64(lda * n, -1, 1, 43), lda)
    A = np.asarray(call[7], dt)
    dx = up(ctx, x, dt)
    dA = up(ctx, A, dt)
    getattr(ctx, r)(m, n, 0.75, dx.offset(1), 1, up(ctx, call[5], dt), 1, dA, lda)
    got = dA.to_host()
    ref = orc.sger_ld(m, n, 0.75, np.asarray(x[1:], dt), 1, np.asarray(call[5], dt), 1, A, lda)
    idx = region(m, n, lda)
    eps, threshold = PREC[r][1], PREC[r][2]
    xv, yv = np.asarray(x[1:], dt).astype(np.float64), np.asarray(call[5], dt).astype(np.float64)
    bound = eps * (np.abs(0.75 * np.outer(xv, yv)).ravel() + np.abs(A.astype(np.float64)[idx]))
    assert np.all(np.abs(got[idx].astype(np.float64) - ref[idx]) <= threshold * bound)
    keep = np.ones(len(A), bool)
    keep[idx] = False
    assert bits_equal(got[keep], A[keep])
