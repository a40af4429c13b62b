"""GPU parity of strmv / dtrmv (y <- op(T) x, out of place) through the C ABI
against the oracle's long-double restatement, under the reference's metric
(tests/strmv/helpers.js): |y - y_ref| <= eps (n+1) sum_j |op(T)(i, j) x(j)|,
eps = 2^-23 with factor <= 2 (the reference's THRESHOLD) in fp32, 2^-48
with factor <= 1 in fp64. Edge cases are held exactly (the reference's
assert.deepEqual) and IEEE regressions to the same NaN / Inf positions; the
unstored triangle (and the diagonal under unit) holds NaN in the larger
cases and must never reach y, y's slots hold NaN before the call (written,
never read) and its stride gaps come back bit-identical. Scenarios follow
tests/strmv/src/test.strmv.js and tests/dtrmv/src/test.dtrmv.js; dtrmv's
"f32 exponent range" inputs are checked in f64's range. Cases are written in
the reference's terms and mapped onto the column-major C ABI as the JS layer
does (tests/refcases.py)."""
import numpy as np
import pytest

from oracle import orc
from tests import refcases as rc
from tests.helpers import EPS32, EPS_DD, bits_equal

pytestmark = pytest.mark.gpu

PREC = {"strmv": (np.float32, EPS32, 2.0), "dtrmv": (np.float64, EPS_DD, 1.0)}


def up(ctx, a, dt):
    a = np.asarray(a, dt)
    return ctx.upload(a if a.size else np.zeros(1, dt))


def run(ctx, r, call):
    dt = PREC[r][0]
    uplo, trans, diag, n, A, lda, x, incx, y, incy = call
    dy = up(ctx, y, dt)
    getattr(ctx, r)(uplo, trans, diag, n, up(ctx, A, dt), lda, up(ctx, x, dt), incx, dy, incy)
    return dy.to_host()[: len(y)]


def check(ctx, r, call, exact=False):
    dt, eps, threshold = PREC[r]
    uplo, trans, diag, n, A, lda, x, incx, y, incy = call
    got = run(ctx, r, call)
    ref, ad = orc.strmv_ld(uplo, trans, diag, n, A, lda, x, incx, y, incy)
    if exact:
        assert bits_equal(got, ref.astype(dt))
        return got
    idx = np.arange(n) * incy
    g, rf = got[idx].astype(np.float64), ref[idx]
    assert np.array_equal(np.isnan(g), np.isnan(rf))
    inf = np.isinf(rf)
    assert np.array_equal(g[inf], rf[inf])
    bound = eps * (n + 1) * ad[:n]
    fin = np.isfinite(rf)
    err = np.abs(g[fin] - rf[fin])
    assert np.all((err <= threshold * bound[fin]) | (err == 0))
    gaps = np.ones(len(y), bool)
    gaps[idx] = False
    assert bits_equal(got[gaps], np.asarray(y, dt)[gaps])  # stride gaps untouched
    return got


def case(layout, uplo, trans, diag, n, inc, seeds=(71, 72, 73), pad=0):
    lda = n + pad
    y = orc.random_f64((n - 1) * inc + 1, -1, 1, seeds[2])
    y[np.arange(n) * inc] = np.nan  # output only: never read
    return dict(layout=layout, uplo=uplo, trans=trans, diag=diag, n=n, A=orc.random_f64(n * lda, -1, 1, seeds[0]),
                lda=lda, x=orc.random_f64((n - 1) * inc + 1, -1, 1, seeds[1]), incx=inc, y=y, incy=inc)


@pytest.mark.parametrize("r", ["strmv", "dtrmv"])
@pytest.mark.parametrize("cm", [False, True])
def test_edge_cases_exact(ctx, r, cm):
    # test.strmv.js:107-142, 218-256 (deepEqual against stdlib); dtrmv the same
    for c in rc.load(r, cm):
        check(ctx, r, rc.trmv_call(c, PREC[r][0]), exact=True)


@pytest.mark.parametrize("r", ["strmv", "dtrmv"])
def test_zero_dimension_leaves_y(ctx, r):
    # test.strmv.js:144-168
    dt = PREC[r][0]
    y = orc.random_f64(4, -1, 1, 9401).astype(dt)
    assert bits_equal(run(ctx, r, (1, 0, 0, 0, np.zeros(0), 1, np.zeros(0), 1, y, 1)), y)


@pytest.mark.parametrize("r", ["strmv", "dtrmv"])
@pytest.mark.parametrize("layout", ["row-major", "column-major"])
@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("trans", ["no-transpose", "transpose"])
@pytest.mark.parametrize("diag", ["non-unit", "unit"])
@pytest.mark.parametrize("inc", [1, 3])
def test_large_n_paths(ctx, r, layout, uplo, trans, diag, inc):
    # test.strmv.js:170-216 (N = 600 over layout x uplo x trans x diag x inc),
    # test.dtrmv.js:188-242 (split-K and packed x); lda = n + 3 for dtrmv
    c = case(layout, uplo, trans, diag, 600, inc, pad=3 if r == "dtrmv" else 0)
    check(ctx, r, rc.trmv_call(c, PREC[r][0]))


@pytest.mark.parametrize("r", ["strmv", "dtrmv"])
@pytest.mark.parametrize("layout", ["row-major", "column-major"])
@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("trans", ["no-transpose", "transpose"])
@pytest.mark.parametrize("n", [7, 300])
def test_zero_x_entries_skip_their_column(ctx, r, layout, uplo, trans, n):
    # test.strmv.js:258-306, test.dtrmv.js:394-442: Infinity at (3,1), (1,3),
    # (n-1,0), (0,n-1), NaN on the diagonal at x's zero entry 1; only the
    # column form skips, so NaN reaches y in the dot form
    dt = PREC[r][0]
    A = orc.random_f64(n * n, -1, 1, 1)
    for i, j in ((3, 1), (1, 3), (n - 1, 0), (0, n - 1)):
        A[i * n + j] = np.inf
    A[1 * n + 1] = np.nan
    x = orc.random_f64(n, -1, 1, 2)
    x[1] = x[n - 1] = 0.0
    c = dict(layout=layout, uplo=uplo, trans=trans, diag="non-unit", n=n, A=A, lda=n, x=x, incx=1,
             y=orc.random_f64(n, -1, 1, 3), incy=1)
    check(ctx, r, rc.trmv_call(c, dt))


def test_dtrmv_exactness(ctx):
    # test.dtrmv.js:283-302: integer-valued inputs give the exact product in
    # every form; the gaps of a strided y are never written
    n = 9
    for uplo in (1, 2):
        for trans in (0, 1):
            for diag in (0, 1):
                A = np.round(orc.random_f64(n * n, -8, 8, 11))
                x = np.round(orc.random_f64(3 * (n - 1) + 1, -8, 8, 12))
                y = orc.random_f64(3 * (n - 1) + 1, -1, 1, 13) * np.pi
                check(ctx, "dtrmv", (uplo, trans, diag, n, A, n, x, 3, y, 3), exact=True)
    full = lambda size, s: orc.random_f64(size, -1, 1, s) * np.pi  # noqa: E731
    check(ctx, "dtrmv", (1, 1, 0, 5, full(25, 980), 5, full(13, 981), 3, full(13, 982), 3))


@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("n", [7, 300])
def test_dtrmv_ieee_special_values(ctx, uplo, n):
    # test.dtrmv.js:304-345: Infinity in the stored triangle reaches y, NaN in
    # the unstored one never does
    rr, cc = (4, 1) if uplo == "lower" else (1, 4)
    for trans in ("no-transpose", "transpose"):
        c = case("row-major", uplo, trans, "non-unit", n, 1, seeds=(1, 2, 3))
        c["A"][rr * n + cc] = np.inf
        c["A"][cc * n + rr] = np.nan
        got = check(ctx, "dtrmv", rc.trmv_call(c, np.float64))
        assert np.isinf(got).any() and not np.isnan(got).any()


@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("n", [7, 300])
def test_dtrmv_f64_exponent_range(ctx, uplo, n):
    # the inputs of test.dtrmv.js:347-392 in f64's range: 1e300 and 1e-50 read
    # as they are, a product past 3.4e38 stays finite
    for trans in ("no-transpose", "transpose"):
        c = case("row-major", uplo, trans, "non-unit", n, 1, seeds=(1, 2, 3))
        c["A"][2 * n + 2], c["A"][3 * n + 3] = 1e300, 1e-50
        got = check(ctx, "dtrmv", rc.trmv_call(c, np.float64))
        assert np.all(np.isfinite(got)) and np.abs(got).max() > 1e299
        c = case("row-major", uplo, trans, "non-unit", n, 1, seeds=(1, 2, 3))
        c["x"][2] = 1e30
        c["A"][2 * n + 2] = 1e10
        got = check(ctx, "dtrmv", rc.trmv_call(c, np.float64))
        assert np.all(np.isfinite(got)) and np.abs(got).max() > 3.4e38


@pytest.mark.parametrize("r", ["strmv", "dtrmv"])
@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("trans", [0, 1])
@pytest.mark.parametrize("diag", [0, 1])
@pytest.mark.parametrize("n,lda", [(4096, 4096), (3001, 3003), (1025, 1028), (129, 129)])
def test_large_unstored_nan(ctx, r, uplo, trans, diag, n, lda):
    # many row chunks and panels, odd lda (element loads), a last chunk of
    # one row, panels crossing the diagonal; the unstored triangle (and the
    # diagonal under unit) holds NaN
    dt = PREC[r][0]
    A = orc.random_f64(lda * n, -1, 1, 81)
    i, j = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
    unstored = (i < j) if uplo == 1 else (i > j)
    if diag:
        unstored |= i == j
    A[(i + j * lda)[unstored]] = np.nan
    y = np.full(n, np.nan)
    call = (uplo, trans, diag, n, A.astype(dt), lda, orc.random_f64(n, -1, 1, 82).astype(dt), 1, y.astype(dt), 1)
    got = check(ctx, r, call)
    assert np.all(np.isfinite(got))
