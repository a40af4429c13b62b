"""GPU parity of ssyr / dsyr and ssyr2 / dsyr2 (symmetric rank-1 / rank-2
updates of one triangle) through the C ABI against the oracle's long-double
restatement, under the reference's metric (tests/ssyr2/helpers.js, the same
shape for ssyr): |A - A_ref| <= eps (|alpha x_i y_j| + |alpha y_i x_j| +
|A_in|) on the triangle, eps = 2^-23 with factor <= 2 (the reference's
THRESHOLD) in fp32, 2^-48 with factor <= 1 in fp64; the other triangle and
lda padding bit-identical. Edge cases are held exactly and IEEE regressions
to the same NaN / Inf positions, as the reference's tests do. Scenarios
follow tests/{ssyr,ssyr2,dsyr,dsyr2}/src/test.*.js; the fp64 "f32 exponent
range" inputs are checked in f64's range. Cases are written in the
reference's terms and mapped onto the column-major C ABI as the JS layer
does (tests/refcases.py)."""
import numpy as np
import pytest

from oracle import orc
from tests import refcases as rc
from tests.helpers import EPS32, EPS_DD, bits_equal

pytestmark = pytest.mark.gpu

PREC = {"ssyr": (np.float32, EPS32, 2.0), "ssyr2": (np.float32, EPS32, 2.0),
        "dsyr": (np.float64, EPS_DD, 1.0), "dsyr2": (np.float64, EPS_DD, 1.0)}


def up(ctx, a, dt):
    a = np.asarray(a, dt)
    return ctx.upload(a if a.size else np.zeros(1, dt))


def split(call):
    """(uplo, n, alpha, x, incx, y or None, incy, A, lda) of a syr / syr2 call."""
    if len(call) == 7:
        uplo, n, alpha, x, incx, A, lda = call
        return uplo, n, alpha, x, incx, None, 1, A, lda
    return call


def run(ctx, r, call):
    dt = PREC[r][0]
    uplo, n, alpha, x, incx, y, incy, A, lda = split(call)
    dA = up(ctx, A, dt)
    if y is None:
        getattr(ctx, r)(uplo, n, alpha, up(ctx, x, dt), incx, dA, lda)
    else:
        getattr(ctx, r)(uplo, n, alpha, up(ctx, x, dt), incx, up(ctx, y, dt), incy, dA, lda)
    return dA.to_host()[: len(A)]


def tri_index(uplo, n, lda):
    i, j = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
    mask = (i >= j) if uplo == 1 else (i <= j)
    return (i + j * lda)[mask], i[mask], j[mask]


def check(ctx, r, call, exact=False):
    dt, eps, threshold = PREC[r]
    uplo, n, alpha, x, incx, y, incy, A, lda = split(call)
    got = run(ctx, r, call)
    ref = orc.ssyr2_ld(uplo, n, alpha, x, incx, y, incy, A, lda)
    if exact:
        assert bits_equal(got, ref.astype(dt))
        return got
    idx, ii, jj = tri_index(uplo, n, lda)
    g, rf = got[idx].astype(np.float64), ref[idx]
    assert np.array_equal(np.isnan(g), np.isnan(rf))
    inf = np.isinf(rf)
    assert np.array_equal(g[inf], rf[inf])
    xv = np.asarray(x, np.float64)[np.arange(n) * incx]
    yv = xv if y is None else np.asarray(y, np.float64)[np.arange(n) * incy]
    with np.errstate(invalid="ignore", over="ignore"):
        terms = np.abs(alpha * xv[ii] * yv[jj])
        if y is not None:
            terms = terms + np.abs(alpha * yv[ii] * xv[jj])
        bound = eps * (terms + np.abs(np.asarray(A, np.float64)[idx]))
    fin = np.isfinite(rf)
    err = np.abs(g[fin] - rf[fin])
    assert np.all((err <= threshold * bound[fin]) | (err == 0))
    keep = np.ones(len(A), bool)
    keep[idx] = False
    assert bits_equal(got[keep], np.asarray(A, dt)[keep])  # other triangle, padding
    return got


def case(r, layout, uplo, n, inc, alpha=1.5, seeds=(211, 212, 213), lda=None):
    ln = (n - 1) * inc + 1
    c = dict(layout=layout, uplo=uplo, n=n, alpha=alpha, x=orc.random_f64(ln, -1, 1, seeds[0]), incx=inc,
             A=orc.random_f64(n * (lda or n), -1, 1, seeds[2]), lda=lda or n)
    if r.endswith("2"):
        c.update(y=orc.random_f64(ln, -1, 1, seeds[1]), incy=inc)
    return c


ROUTINES = ["ssyr", "ssyr2", "dsyr", "dsyr2"]


@pytest.mark.parametrize("r", ROUTINES)
@pytest.mark.parametrize("cm", [False, True])
def test_edge_cases_exact(ctx, r, cm):
    # test.ssyr.js:81-109, 130-163 (deepEqual against stdlib); the others the same
    for c in rc.load(r, cm):
        check(ctx, r, rc.syr_call(c, PREC[r][0]), exact=True)


@pytest.mark.parametrize("r", ROUTINES)
def test_zero_dimension_leaves_a(ctx, r):
    # test.ssyr.js:111-128
    dt = PREC[r][0]
    A = orc.random_f64(16, -1, 1, 9201).astype(dt)
    x = orc.random_f64(4, -1, 1, 9202)
    call = (1, 0, 1.5, x, 1, A, 4) if not r.endswith("2") else (1, 0, 1.5, x, 1, x, 1, A, 4)
    assert bits_equal(run(ctx, r, call), A)


@pytest.mark.parametrize("r", ROUTINES)
@pytest.mark.parametrize("layout", ["row-major", "column-major"])
@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("n", [7, 300])
def test_zero_vector_entries_skip_their_row(ctx, r, layout, uplo, n):
    # test.ssyr.js:165-209, test.ssyr2.js:202-250: zeros beside Infinity and
    # NaN, stride 2 (syr2 skips only where both vectors are zero)
    c = case(r, layout, uplo, n, 2, seeds=(1, 2, 3))
    x = c["x"]
    for i in (0, 3, 5):
        x[i * 2] = 0
    x[1 * 2], x[6 * 2] = np.inf, -np.inf
    if "y" in c:
        y = c["y"]
        for i in (1, 3, 6):
            y[i * 2] = 0
        y[5 * 2] = np.nan
    else:
        x[4 * 2] = np.nan
    got = check(ctx, r, rc.syr_call(c, PREC[r][0]))
    assert np.isnan(got).any() and np.isinf(got).any()


@pytest.mark.parametrize("r", ROUTINES)
def test_alpha_zero_leaves_a(ctx, r):
    # test.ssyr.js:211-230: x holds Infinity and NaN, never read
    dt = PREC[r][0]
    c = case(r, "row-major", "lower", 6, 1, alpha=0.0, seeds=(1, 2, 3))
    c["x"][1], c["x"][3] = np.inf, np.nan
    A = np.asarray(c["A"], dt)
    assert bits_equal(run(ctx, r, rc.syr_call(c, dt)), A)


@pytest.mark.parametrize("r", ROUTINES)
@pytest.mark.parametrize("N,inc", [(600, 1), (600, 3), (1100, 8)])
@pytest.mark.parametrize("layout", ["row-major", "column-major"])
@pytest.mark.parametrize("uplo", ["lower", "upper"])
def test_multi_chunk_and_strides(ctx, r, N, inc, layout, uplo):
    # test.dsyr.js:152-200, test.dsyr2.js:185-237: lda = n + 3
    check(ctx, r, rc.syr_call(case(r, layout, uplo, N, inc, lda=N + 3), PREC[r][0]))


@pytest.mark.parametrize("r", ["dsyr", "dsyr2"])
@pytest.mark.parametrize("uplo", ["lower", "upper"])
@pytest.mark.parametrize("n", [7, 300])
def test_fp64_ieee_special_values(ctx, r, uplo, n):
    # test.dsyr.js:255-284, test.dsyr2.js:318-351: Infinity in x, NaN in y
    # (dsyr: in x) propagate as in real f64
    c = case(r, "row-major", uplo, n, 1, seeds=(1, 2, 3))
    c["x"][2] = np.inf
    if "y" in c:
        c["y"][5] = np.nan
    else:
        c["x"][5] = np.nan
    got = check(ctx, r, rc.syr_call(c, np.float64))
    assert np.isnan(got).any() and np.isinf(got).any()


@pytest.mark.parametrize("r", ["dsyr", "dsyr2"])
@pytest.mark.parametrize("n", [7, 300])
def test_fp64_exponent_range(ctx, r, n):
    # the inputs of the "f32 exponent range" regressions (test.dsyr.js:286-353,
    # test.dsyr2.js:353-428) in f64's range: 1e300 / 1e-50 read as they are,
    # a product past 3.4e38 stays finite
    c = case(r, "row-major", "lower", n, 1, seeds=(1, 2, 3))
    c["x"][2], c["x"][4] = 1e150, 1e-50
    c["A"][0] = -1e300
    got = check(ctx, r, rc.syr_call(c, np.float64))
    assert np.all(np.isfinite(got)) and np.abs(got).max() > 1e299
    c = case(r, "row-major", "lower", n, 1, alpha=1e10, seeds=(1, 2, 3))
    c["x"][2] = 1e30
    got = check(ctx, r, rc.syr_call(c, np.float64))
    assert np.all(np.isfinite(got)) and np.abs(got).max() > 3.4e38


@pytest.mark.parametrize("r", ROUTINES)
@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("n,lda", [(4096, 4096), (3001, 3003), (1025, 1028)])
def test_large_and_odd(ctx, r, uplo, n, lda):
    # whole and diagonal columns of many row blocks; odd lda takes element
    # accesses; 1025 rows leave one row in the last block
    dt = PREC[r][0]
    x = orc.random_f64(n, -1, 1, 51)
    A = orc.random_f64(lda * n, -1, 1, 53)
    call = ((uplo, n, 0.75, x, 1, A, lda) if not r.endswith("2")
            else (uplo, n, 0.75, x, 1, orc.random_f64(n, -1, 1, 52), 1, A, lda))
    check(ctx, r, tuple(np.asarray(v, dt) if isinstance(v, np.ndarray) else v for v in call))
