"""GPU parity of ssymv / dsymv through the C ABI against the oracle's
long-double restatement, under the reference's metric (tests/ssymv/helpers.js):
|y - y_ref| <= eps ((n+2) |alpha| sum|S x| + 2 |beta| |y_in|), eps = 2^-23
with factor <= 2 (the reference's THRESHOLD) in fp32, 2^-48 with factor <= 1
in fp64. Edge cases are held exactly (the reference's assert.deepEqual) and
IEEE regressions to the same NaN / Inf positions; the unstored triangle holds
NaN in the larger cases and must never reach y. Scenarios follow
tests/ssymv/src/test.ssymv.js and tests/dsymv/src/test.dsymv.js; dsymv's
"f32 exponent range" inputs are checked in f64's range. Cases are written in
the reference's terms and mapped onto the column-major C ABI as the JS layer
does (tests/refcases.py)."""
import numpy as np
import pytest

from oracle import orc
from tests import refcases as rc
from tests.helpers import EPS32, EPS_DD, bits_equal

pytestmark = pytest.mark.gpu

PREC = {"ssymv": (np.float32, EPS32, 2.0), "dsymv": (np.float64, EPS_DD, 1.0)}


def up(ctx, a, dt):
    a = np.asarray(a, dt)
    return ctx.upload(a if a.size else np.zeros(1, dt))


def run(ctx, r, call):
    dt = PREC[r][0]
    uplo, n, alpha, A, lda, x, incx, beta, y, incy = call
    dy = up(ctx, y, dt)
    getattr(ctx, r)(uplo, n, alpha, up(ctx, A, dt), lda, up(ctx, x, dt), incx, beta, dy, incy)
    return dy.to_host()[: len(y)]


def check(ctx, r, call, exact=False, ref_y=None):
    dt, eps, threshold = PREC[r]
    uplo, n, alpha, A, lda, x, incx, beta, y, incy = call
    got = run(ctx, r, call)
    yr = np.asarray(y if ref_y is None else ref_y, np.float64)
    ref, ad = orc.ssymv_ld(uplo, n, alpha, A, lda, x, incx, beta, yr, incy)
    if exact:
        assert bits_equal(got, ref.astype(dt))
        return got
    idx = np.arange(n) * incy
    g, rf = got[idx].astype(np.float64), ref[idx]
    assert np.array_equal(np.isnan(g), np.isnan(rf))
    inf = np.isinf(rf)
    assert np.array_equal(g[inf], rf[inf])
    yin = np.abs(yr[idx]) if beta != 0 else 0.0
    bound = np.broadcast_to(eps * ((n + 2) * abs(alpha) * ad[:n] + 2 * abs(beta) * yin), g.shape)
    fin = np.isfinite(rf)
    err = np.abs(g[fin] - rf[fin])
    assert np.all((err <= threshold * bound[fin]) | (err == 0))
    gaps = np.ones(len(y), bool)
    gaps[idx] = False
    assert bits_equal(got[gaps], np.asarray(y, dt)[gaps])  # stride gaps untouched
    return got


def case(layout, uplo, n, inc, beta, alpha=1.5, seeds=(31, 32, 33), pad=0):
    lda = n + pad
    return dict(layout=layout, uplo=uplo, n=n, alpha=alpha, A=orc.random_f64(n * lda, -1, 1, seeds[0]), lda=lda,
                x=orc.random_f64((n - 1) * inc + 1, -1, 1, seeds[1]), incx=inc, beta=beta,
                y=orc.random_f64((n - 1) * inc + 1, -1, 1, seeds[2]), incy=inc)


@pytest.mark.parametrize("r", ["ssymv", "dsymv"])
@pytest.mark.parametrize("cm", [False, True])
def test_edge_cases_exact(ctx, r, cm):
    # test.ssymv.js:110-145, 219-256 (deepEqual against stdlib); dsymv the same
    for c in rc.load(r, cm):
        check(ctx, r, rc.symv_call(c, PREC[r][0]), exact=True)


@pytest.mark.parametrize("r", ["ssymv", "dsymv"])
def test_zero_dimension_leaves_y(ctx, r):
    # test.ssymv.js:147-171
    dt = PREC[r][0]
    y = orc.random_f64(4, -1, 1, 9301).astype(dt)
    assert bits_equal(run(ctx, r, (1, 0, 1.5, np.zeros(0), 1, np.zeros(0), 1, 0.5, y, 1)), y)


@pytest.mark.parametrize("r", ["ssymv", "dsymv"])
@pytest.mark.parametrize("layout", ["row-major", "column-major"])
@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("N,inc,beta", [(600, 1, 0.0), (600, 3, 0.75), (256, 1, 0.75), (257, 1, 0.75),
                                        (600, 1, 0.75), (600, 3, 0.0)])
def test_many_tile_paths(ctx, r, layout, uplo, N, inc, beta):
    # test.ssymv.js:173-217 (N = 600, beta 0 / 0.75, inc 1 / 3) and
    # test.dsymv.js:191-248 (256, 257, 600; lda = n + 3)
    c = case(layout, uplo, N, inc, beta, pad=3 if N != 600 or r == "dsymv" else 0)
    check(ctx, r, rc.symv_call(c, PREC[r][0]))


@pytest.mark.parametrize("r", ["ssymv", "dsymv"])
@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("n", [7, 300])
@pytest.mark.parametrize("beta", [0.0, 0.5])
def test_alpha_zero_reads_neither_a_nor_x(ctx, r, uplo, n, beta):
    # test.ssymv.js:258-297: NaN / Inf in A and x never read; beta = 0
    # ignores NaN in y
    dt = PREC[r][0]
    A = orc.random_f64(n * n, -1, 1, 1)
    A[3 * n + 1], A[1 * n + 3], A[2 * n + 2] = np.nan, np.inf, -np.inf
    x = orc.random_f64(n, -1, 1, 2)
    x[5] = np.inf
    y = orc.random_f64(n, -1, 1, 3)
    if beta == 0:
        y[0] = np.nan
    c = dict(uplo=uplo, n=n, alpha=0.0, A=A, lda=n, x=x, incx=1, beta=beta, y=y, incy=1)
    got = run(ctx, r, rc.symv_call(c, dt))
    want = np.zeros(n, dt) if beta == 0 else (dt(beta) * np.asarray(y, dt)).astype(dt)
    assert bits_equal(got, want)


def test_dsymv_exactness(ctx):
    # test.dsymv.js:289-331: alpha = 0, beta = 1 returns y bit for bit; the
    # gaps of a strided y are never written
    n = 6
    full = lambda size, s: orc.random_f64(size, -1, 1, s) * np.pi  # noqa: E731
    y = full(n, 1040)
    assert bits_equal(run(ctx, "dsymv", (1, n, 0.0, full(n * n, 1), n, full(n, 2), 1, 1.0, y, 1)), y)
    for beta in (0.0, 0.5):
        check(ctx, "dsymv", (2, n, 1.5, full(n * n, 3), n, full(16, 4), 3, beta, full(16, 5), 3))


@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("n", [7, 300])
def test_dsymv_ieee_special_values(ctx, uplo, n):
    # test.dsymv.js:333-376: Infinity in the stored triangle reaches both its
    # row and its mirror; NaN in the unstored one never does
    rr, cc = (4, 1) if uplo == "lower" else (1, 4)
    c = case("row-major", uplo, n, 1, 0.5, seeds=(1, 2, 3))
    c["A"][rr * n + cc] = np.inf
    c["A"][cc * n + rr] = np.nan
    got = check(ctx, "dsymv", rc.symv_call(c, np.float64))
    assert np.isinf(got).any() and not np.isnan(got).any()


@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("n", [7, 300])
def test_dsymv_f64_exponent_range(ctx, uplo, n):
    # the inputs of test.dsymv.js:378-422 in f64's range
    c = case("row-major", uplo, n, 1, 0.5, seeds=(1, 2, 3))
    c["A"][2 * n + 2], c["A"][3 * n + 3] = 1e300, 1e-50
    c["y"][1] = -1e300
    got = check(ctx, "dsymv", rc.symv_call(c, np.float64))
    assert np.all(np.isfinite(got)) and np.abs(got).max() > 1e299
    c = case("row-major", uplo, n, 1, 0.5, alpha=1e10, seeds=(1, 2, 3))
    c["x"][5] = 1e30
    got = check(ctx, "dsymv", rc.symv_call(c, np.float64))
    assert np.all(np.isfinite(got)) and np.abs(got).max() > 3.4e38


@pytest.mark.parametrize("r", ["ssymv", "dsymv"])
@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("n,lda", [(4096, 4096), (3001, 3003), (1025, 1028), (129, 129)])
def test_large_unstored_nan(ctx, r, uplo, n, lda):
    # many row chunks and panels, odd lda (element loads), a last chunk of
    # one row, panels crossing the diagonal; the unstored triangle holds NaN
    dt = PREC[r][0]
    A = orc.random_f64(lda * n, -1, 1, 61)
    i, j = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
    unstored = (i < j) if uplo == 1 else (i > j)
    A[(i + j * lda)[unstored]] = np.nan
    call = (uplo, n, 0.75, A.astype(dt), lda, orc.random_f64(n, -1, 1, 62).astype(dt), 1, -1.25,
            orc.random_f64(n, -1, 1, 63).astype(dt), 1)
    got = check(ctx, r, call)
    assert np.all(np.isfinite(got))
