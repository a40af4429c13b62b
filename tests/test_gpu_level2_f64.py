"""GPU parity of dgemv (native fp64 on the sgemv kernels) through the C ABI
against the oracle's long-double restatement, under the reference's metric
(tests/dgemv/helpers.js): |y - y_ref| <= eps ((terms+1) |alpha| sum|a x| +
|beta||y_in|), eps = 2^-48 (factor <= 1 here; the reference allows 5). The
reference's edge cases are held to exact equality, as its test does
(assert.deepEqual against stdlib), and the IEEE regressions to the same NaN /
Inf positions. The scenarios follow tests/dgemv/src/test.dgemv.js; its
"f32 exponent range" regression describes double-double's range, so here
its inputs are checked in f64's range instead. Cases are written in the
reference's terms and mapped onto the column-major C ABI as the JS layer
does (tests/refcases.py)."""
import numpy as np
import pytest

from oracle import orc
from tests import refcases as rc
from tests.helpers import EPS_DD, bits_equal

pytestmark = pytest.mark.gpu

F64 = np.float64


def up(ctx, a):
    a = np.asarray(a, F64)
    return ctx.upload(a if a.size else np.zeros(1, F64))


def run(ctx, call):
    trans, m, n, alpha, A, lda, x, incx, beta, y, incy = call
    dy = up(ctx, y)
    ctx.dgemv(trans, m, n, alpha, up(ctx, A), lda, up(ctx, x), incx, beta, dy, incy)
    return dy.to_host()[: len(y)] if len(y) else np.zeros(0, F64)


def check(ctx, call, exact=False, ref_y=None):
    """ref_y: the y the oracle sees (beta = 0 cases pass zeros)."""
    trans, m, n, alpha, A, lda, x, incx, beta, y, incy = call
    got = run(ctx, call)
    yr = np.asarray(y if ref_y is None else ref_y, F64)
    ref, ad = orc.sgemv_ld(trans, m, n, alpha, A, lda, x, incx, beta, yr, incy)
    ln = n if trans else m
    idx = np.arange(ln) * incy
    if exact:
        assert bits_equal(got, ref)
        return got
    g, r = got[idx], ref[idx]
    assert np.array_equal(np.isnan(g), np.isnan(r))
    inf = np.isinf(r)
    assert np.array_equal(g[inf], r[inf])
    fin = np.isfinite(r)
    terms = m if trans else n
    yin = np.abs(yr[idx]) if beta != 0 else 0.0
    bound = EPS_DD * ((terms + 1) * abs(alpha) * ad[:ln] + abs(beta) * yin)
    bound = np.broadcast_to(bound, g.shape)  # ad: one entry per output element
    err = np.abs(g[fin] - r[fin])
    assert np.all((err <= bound[fin]) | (err == 0))
    keep = np.ones(len(y), bool)
    keep[idx] = False
    assert bits_equal(got[keep], np.asarray(y, F64)[keep])  # stride gaps untouched
    return got


def at(n, i, j):
    return i * n + j


@pytest.mark.parametrize("cm", [False, True])
def test_edge_cases_exact(ctx, cm):
    # test.dgemv.js:130-169, 344-383 (deepEqual against stdlib)
    for c in rc.load("dgemv", cm):
        check(ctx, rc.gemv_call(c, F64), exact=True)


def test_zero_dimension_leaves_y(ctx):
    # test.dgemv.js:171-218: the contraction dimension 0 with beta = 0.5
    y = orc.random_f64(4, -1, 1, 9001)
    assert bits_equal(run(ctx, (0, 4, 0, 1.5, np.zeros(0), 4, np.zeros(0), 1, 0.5, y, 1)), y)
    assert bits_equal(run(ctx, (1, 0, 4, 1.5, np.zeros(0), 1, np.zeros(0), 1, 0.5, y, 1)), y)


@pytest.mark.parametrize("trans,layout,K,N,inc,beta", [
    ("transpose", "row-major", 600, 70, 1, 0.75), ("transpose", "row-major", 600, 70, 3, 0.75),
    ("transpose", "row-major", 600, 70, 1, 0.0), ("no-transpose", "column-major", 600, 70, 2, 0.75),
    ("transpose", "row-major", 256, 70, 1, 0.75), ("transpose", "row-major", 257, 130, 1, 0.75)])
def test_split_k_transpose(ctx, trans, layout, K, N, inc, beta):
    # test.dgemv.js:220-288: the contraction split several ways; beta = 0
    # with NaN already in y
    no = trans == "no-transpose"
    m, n = (N, K) if no else (K, N)
    lda = (n if layout == "row-major" else m) + 3
    outer = m if layout == "row-major" else n
    y = orc.random_f64((N - 1) * inc + 1, -1, 1, 307)
    if beta == 0:
        y[np.arange(N) * inc] = np.nan
    c = dict(layout=layout, trans=trans, m=m, n=n, alpha=1.5, A=orc.random_f64(outer * lda, -1, 1, 301),
             lda=lda, x=orc.random_f64((K - 1) * inc + 1, -1, 1, 303), incx=inc, beta=beta, y=y,
             incy=inc)
    call = rc.gemv_call(c, F64)
    got = check(ctx, call, ref_y=np.where(np.isnan(call[9]), 0.0, call[9]) if beta == 0 else None)
    assert np.all(np.isfinite(got[np.arange(N) * inc]))


@pytest.mark.parametrize("n,m,inc,beta", [(600, 70, 1, 0.75), (600, 70, 2, 0.75), (600, 70, 1, 0.0),
                                          (256, 33, 1, 0.75), (319, 33, 3, 0.75)])
def test_long_rows_no_transpose(ctx, n, m, inc, beta):
    # test.dgemv.js:290-342 (row-major, so the column-major transposed form)
    lda = n + 3
    y = orc.random_f64((m - 1) * inc + 1, -1, 1, 317)
    if beta == 0:
        y[np.arange(m) * inc] = np.nan
    c = dict(trans="no-transpose", m=m, n=n, alpha=1.5, A=orc.random_f64(m * lda, -1, 1, 311), lda=lda,
             x=orc.random_f64((n - 1) * inc + 1, -1, 1, 313), incx=inc, beta=beta, y=y, incy=inc)
    call = rc.gemv_call(c, F64)
    check(ctx, call, ref_y=np.where(np.isnan(call[9]), 0.0, call[9]) if beta == 0 else None)


@pytest.mark.parametrize("trans", [0, 1])
def test_quick_return_and_stride_gaps(ctx, trans):
    # test.dgemv.js:385-430: alpha = 0, beta = 1 returns y bit for bit; the
    # gaps of a strided y are never written
    n = 5
    full = lambda size, s: orc.random_f64(size, -1, 1, s) * np.pi  # noqa: E731
    y = full(n, 960)
    assert bits_equal(run(ctx, (trans, n, n, 0.0, full(n * n, 1), n, full(n, 2), 1, 1.0, y, 1)), y)
    for beta in (0.0, 0.5):
        check(ctx, (trans, n, n, 1.5, full(n * n, 3), n, full(13, 4), 3, beta, full(13, 5), 3))


@pytest.mark.parametrize("trans", ["no-transpose", "transpose"])
@pytest.mark.parametrize("n", [7, 300])
def test_ieee_special_values(ctx, trans, n):
    # test.dgemv.js:432-476: Inf / NaN in A and x propagate; beta = 0 ignores
    # NaN / Inf already in y
    A = orc.random_f64(n * n, -1, 1, 1)
    A[at(n, 1, 2)], A[at(n, 3, 4)] = np.inf, np.nan
    x = orc.random_f64(n, -1, 1, 2)
    x[5] = -np.inf
    y = orc.random_f64(n, -1, 1, 3)
    y[0], y[6] = np.nan, np.inf
    c = dict(trans=trans, m=n, n=n, alpha=1.5, A=A, lda=n, x=x, incx=1, beta=0.0, y=y, incy=1)
    got = check(ctx, rc.gemv_call(c, F64), ref_y=np.zeros(n))
    assert np.isnan(got).any()


@pytest.mark.parametrize("trans", ["no-transpose", "transpose"])
@pytest.mark.parametrize("n", [7, 300])
def test_f64_exponent_range(ctx, trans, n):
    # the inputs of test.dgemv.js:478-551 in f64's range: 1e300, 1e-50 and
    # -1e300 are read as they are, and a result past 3.4e38 stays finite
    A = orc.random_f64(n * n, -1, 1, 1)
    A[at(n, 1, 2)], A[at(n, 3, 4)] = 1e300, 1e-50
    x = orc.random_f64(n, -1, 1, 2)
    x[6] = 1e-50
    y = orc.random_f64(n, -1, 1, 3)
    y[0] = -1e300
    c = dict(trans=trans, m=n, n=n, alpha=1.5, A=A, lda=n, x=x, incx=1, beta=0.5, y=y, incy=1)
    got = check(ctx, rc.gemv_call(c, F64))
    assert np.all(np.isfinite(got)) and np.abs(got).max() > 1e299
    x = orc.random_f64(n, -1, 1, 2)
    x[5] = 1e30
    c = dict(c, alpha=1e10, A=orc.random_f64(n * n, -1, 1, 1), x=x, y=orc.random_f64(n, -1, 1, 3))
    got = check(ctx, rc.gemv_call(c, F64))
    assert np.all(np.isfinite(got)) and np.abs(got).max() > 3.4e38


@pytest.mark.parametrize("trans", ["no-transpose", "transpose"])
@pytest.mark.parametrize("n", [7, 300])
@pytest.mark.parametrize("beta", [0.0, 0.5])
def test_alpha_zero_reads_neither_a_nor_x(ctx, trans, n, beta):
    # test.dgemv.js:553-596
    A = orc.random_f64(n * n, -1, 1, 1)
    A[1 * n + 2], A[3 * n + 4] = np.nan, np.inf
    x = orc.random_f64(n, -1, 1, 2)
    x[5] = -np.inf
    y = orc.random_f64(n, -1, 1, 3)
    if beta == 0:
        y[0] = np.nan
    c = dict(trans=trans, m=n, n=n, alpha=0.0, A=A, lda=n, x=x, incx=1, beta=beta, y=y, incy=1)
    got = run(ctx, rc.gemv_call(c, F64))
    want = np.zeros(n) if beta == 0 else beta * y
    assert bits_equal(got, want)


@pytest.mark.parametrize("layout", ["row-major", "column-major"])
@pytest.mark.parametrize("trans", ["no-transpose", "transpose"])
@pytest.mark.parametrize("n", [7, 300])
def test_zero_x_entries_skip_their_column(ctx, layout, trans, n):
    # test.dgemv.js:598-640: NaN / Inf land where reference BLAS puts them
    A = orc.random_f64(n * n, -1, 1, 1)
    A[at(n, 1, 2)], A[at(n, 2, 1)], A[at(n, 4, 0)], A[at(n, 0, 4)] = np.inf, -np.inf, np.nan, np.inf
    x = orc.random_f64(n, -1, 1, 2)
    x[1] = x[4] = 0
    c = dict(layout=layout, trans=trans, m=n, n=n, alpha=1.5, A=A, lda=n, x=x, incx=1, beta=0.5,
             y=orc.random_f64(n, -1, 1, 3), incy=1)
    check(ctx, rc.gemv_call(c, F64))


@pytest.mark.parametrize("trans", [0, 1])
@pytest.mark.parametrize("shape", [(4096, 4096, 4096), (65536, 48, 65536), (48, 65536, 49),
                                   (3001, 2999, 3003), (4097, 1000, 4099), (4096, 1000, 4096)])
def test_large_and_skinny(ctx, trans, shape):
    # the sgemv launch shapes in fp64: one block column / row of output (the
    # contraction split many ways), odd sizes with an odd lda (element
    # loads), x misaligned by one element
    m, n, lda = shape
    A = orc.random_f64(lda * n, -1, 1, 31)
    xl, yl = (n, m) if trans == 0 else (m, n)
    x = orc.random_f64(xl + 1, -1, 1, 32)
    y = orc.random_f64(yl, -1, 1, 33)
    dx = up(ctx, x)
    dy = up(ctx, y)
    ctx.dgemv(trans, m, n, 0.75, up(ctx, A), lda, dx.offset(1), 1, -1.25, dy, 1)
    got = dy.to_host()
    ref, ad = orc.sgemv_ld(trans, m, n, 0.75, A, lda, x[1:], 1, -1.25, y, 1)
    terms = m if trans else n
    bound = EPS_DD * ((terms + 1) * 0.75 * ad + 1.25 * np.abs(y))
    assert np.all(np.abs(got - ref) <= bound)
