"""GPU parity of sgemv through the C ABI against the oracle's long-double
restatement, under the reference's metric (tests/sgemv/helpers.js):
|y - y_ref| <= eps ((terms+1) |alpha| sum|a x| + |beta||y_in|), eps = 2^-23
(factor <= 1 here; the reference allows 4). The reference's edge cases are
held to exact equality, as its test does (assert.deepEqual against stdlib),
and the IEEE regressions to the same NaN / Inf positions. Cases are written
in the reference's terms and mapped onto the column-major C ABI as the JS
layer does (tests/refcases.py)."""
import numpy as np
import pytest

from oracle import orc
from tests import refcases as rc
from tests.helpers import EPS32, bits_equal

pytestmark = pytest.mark.gpu

F32 = np.float32


def up(ctx, a):
    a = np.asarray(a, F32)
    return ctx.upload(a if a.size else np.zeros(1, F32))


def run(ctx, call):
    trans, m, n, alpha, A, lda, x, incx, beta, y, incy = call
    dy = up(ctx, y)
    ctx.sgemv(trans, m, n, alpha, up(ctx, A), lda, up(ctx, x), incx, beta, dy, incy)
    return dy.to_host()[: len(y)] if len(y) else np.zeros(0, F32)


def check(ctx, call, exact=False):
    trans, m, n, alpha, A, lda, x, incx, beta, y, incy = call
    got = run(ctx, call)
    ref, ad = orc.sgemv_ld(*call)
    ln = n if trans else m
    idx = np.arange(ln) * incy
    if exact:
        assert bits_equal(got, ref.astype(F32))
        return got
    terms = m if trans else n
    yin = np.abs(np.asarray(y, np.float64)[idx]) if beta != 0 else 0.0
    bound = EPS32 * ((terms + 1) * abs(alpha) * ad + abs(beta) * yin)
    err = np.abs(got[idx].astype(np.float64) - ref[idx])
    assert np.all((err <= bound) | (err == 0))
    keep = np.ones(len(y), bool)
    keep[idx] = False
    assert bits_equal(got[keep], np.asarray(y, F32)[keep])  # stride gaps untouched
    return got


@pytest.mark.parametrize("cm", [False, True])
def test_edge_cases_exact(ctx, cm):
    for c in rc.load("sgemv", cm):
        check(ctx, rc.gemv_call(c), exact=True)


def test_zero_dimension_leaves_y(ctx):
    # test.sgemv.js:157-202: the contraction dimension 0 with beta = 0.5
    y = orc.random_f32(4, -1, 1, 9001)
    assert bits_equal(run(ctx, (0, 4, 0, 1.5, np.zeros(0), 4, np.zeros(0), 1, 0.5, y, 1)), y)
    assert bits_equal(run(ctx, (1, 0, 4, 1.5, np.zeros(0), 1, np.zeros(0), 1, 0.5, y, 1)), y)


@pytest.mark.parametrize("layout,trans", [("row-major", "transpose"), ("column-major", "no-transpose"),
                                          ("row-major", "no-transpose"), ("column-major", "transpose")])
@pytest.mark.parametrize("beta", [0.0, 0.75])
@pytest.mark.parametrize("inc", [1, 3])
def test_split_k_paths(ctx, layout, trans, beta, inc):
    # test.sgemv.js:204-256: 600 x 300 (several splits of the contraction)
    M, N = 600, 300
    m, n = (M, N) if layout == "row-major" else (N, M)
    no = trans == "no-transpose"
    xl, yl = (n, m) if no else (m, n)
    c = dict(layout=layout, trans=trans, m=m, n=n, alpha=1.5, A=orc.random_f32(m * n, -1, 1, 21),
             lda=n if layout == "row-major" else m, x=orc.random_f32((xl - 1) * inc + 1, -1, 1, 22),
             incx=inc, beta=beta, y=orc.random_f32((yl - 1) * inc + 1, -1, 1, 23), incy=inc)
    check(ctx, rc.gemv_call(c))


@pytest.mark.parametrize("trans", ["no-transpose", "transpose"])
@pytest.mark.parametrize("n", [7, 300])
@pytest.mark.parametrize("beta", [0.0, 0.5])
def test_alpha_zero_reads_neither_a_nor_x(ctx, trans, n, beta):
    # test.sgemv.js:299-342
    A = orc.random_f32(n * n, -1, 1, 1)
    A[1 * n + 2], A[3 * n + 4] = np.nan, np.inf
    x = orc.random_f32(n, -1, 1, 2)
    x[5] = -np.inf
    y = orc.random_f32(n, -1, 1, 3)
    if beta == 0:
        y[0] = np.nan
    c = dict(trans=trans, m=n, n=n, alpha=0.0, A=A, lda=n, x=x, incx=1, beta=beta, y=y, incy=1)
    got = run(ctx, rc.gemv_call(c))
    want = np.zeros(n, F32) if beta == 0 else (np.float32(beta) * y).astype(F32)
    assert bits_equal(got, want)


@pytest.mark.parametrize("layout", ["row-major", "column-major"])
@pytest.mark.parametrize("trans", ["no-transpose", "transpose"])
@pytest.mark.parametrize("n", [7, 300])
def test_zero_x_entries_skip_their_column(ctx, layout, trans, n):
    # test.sgemv.js:344-387: NaN / Inf land where reference BLAS puts them
    at = lambda r, cc: r * n + cc
    A = orc.random_f32(n * n, -1, 1, 1)
    A[at(1, 2)], A[at(2, 1)], A[at(4, 0)], A[at(0, 4)] = np.inf, -np.inf, np.nan, np.inf
    x = orc.random_f32(n, -1, 1, 2)
    x[1] = x[4] = 0
    c = dict(layout=layout, trans=trans, m=n, n=n, alpha=1.5, A=A, lda=n, x=x, incx=1, beta=0.5,
             y=orc.random_f32(n, -1, 1, 3), incy=1)
    call = rc.gemv_call(c)
    got = run(ctx, call).astype(np.float64)
    ref = orc.sgemv_ld(*call)[0]
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isinf(got), np.isinf(ref))
    fin = np.isfinite(ref)
    assert np.allclose(got[fin], ref[fin], rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("trans", [0, 1])
@pytest.mark.parametrize("shape", [(4096, 4096, 4096), (65536, 48, 65536), (48, 65536, 49),
                                   (3001, 2999, 3003), (4097, 1000, 4099), (4096, 1000, 4096)])
def test_large_and_skinny(ctx, trans, shape):
    # one block column / one block row of output (contraction split many
    # ways), odd sizes with an odd lda (element loads), and misaligned x;
    # 4096 / 4097 rows sit either side of the transpose form's switch from
    # 4 to 8 columns per wave
    m, n, lda = shape
    A = orc.random_f32(lda * n, -1, 1, 31)
    xl, yl = (n, m) if trans == 0 else (m, n)
    x = orc.random_f32(xl + 1, -1, 1, 32)
    y = orc.random_f32(yl, -1, 1, 33)
    dx = up(ctx, x)
    dy = up(ctx, y)
    ctx.sgemv(trans, m, n, 0.75, up(ctx, A), lda, dx.offset(1), 1, -1.25, dy, 1)
    got = dy.to_host()
    ref, ad = orc.sgemv_ld(trans, m, n, 0.75, A, lda, x[1:], 1, -1.25, y, 1)
    terms = m if trans else n
    bound = EPS32 * ((terms + 1) * 0.75 * ad + 1.25 * np.abs(y.astype(np.float64)))
    assert np.all(np.abs(got.astype(np.float64) - ref) <= bound)
