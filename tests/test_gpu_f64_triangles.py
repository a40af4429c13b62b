"""GPU parity of dgemmtr and dsyrk (native fp64 on the triangle launch)
through the C ABI, mirroring wgblas's tests/dgemmtr/src/test.dgemmtr.js and
tests/dsyrk/src/test.dsyrk.js regression scenarios.

Every case compares with the oracle's long-double GEMM on the same inputs
under the reference's dgemm bound (eps 2^-48, (k+2) and 3|beta||C|), and
bit-checks that the other triangle and C's ld padding are untouched. The
reference's double-double keeps f32's exponent range; native fp64 does not,
so its "f32 exponent range" regression has no counterpart here.
"""
import numpy as np
import pytest

from oracle import orc
from tests.helpers import bits_equal, untouched_mask
from tests.test_gpu_gemm import check_case, run_gemm

pytestmark = pytest.mark.gpu

F64 = np.float64


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
def test_dgemmtr_large_n_400(ctx, uplo, ta, tb):
    # test.dgemmtr.js:209-275: M = N = 400, K = 8, alpha 1.5, beta 0.5, seeds 0/100/200
    m = n = 400
    k = 8
    check_case(ctx, uplo, ta, tb, m, n, k, 1.5, 0.5, lda=(k if ta else m), ldb=(n if tb else k),
               ldc=m, dtype=F64)


@pytest.mark.parametrize("mn", [(100, 100), (150, 70), (70, 150)])
@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("ta", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
def test_dgemmtr_non_square_and_untouched_triangle(ctx, mn, uplo, ta, tb):
    # test.dgemmtr.js:277-353: K = 9, seeds 51/52/53
    m, n = mn
    k = 9
    check_case(ctx, uplo, ta, tb, m, n, k, 1.5, 0.5, lda=(k if ta else m), ldb=(n if tb else k),
               ldc=m, seeds=(51, 52, 53), dtype=F64)


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("shape", [(1100, 1100, 300), (2100, 1900, 77)])
def test_dgemmtr_large_tier(ctx, uplo, shape):
    m, n, k = shape
    check_case(ctx, uplo, 0, 1, m, n, k, 1.0, 0.25, lda=m, ldb=n, ldc=m + 1, dtype=F64)


@pytest.mark.parametrize("uplo", [1, 2])
def test_dgemmtr_k0_is_beta_c(ctx, uplo):
    # test.dgemmtr.js:355-410: k = 0 gives beta*C on the triangle (exact in
    # fp64), the other triangle unchanged
    m = n = 4
    C = orc.random_f64(m * n, -5, 5, 300 if uplo == 1 else 301)
    got = run_gemm(ctx, uplo, 0, 1, m, n, 0, 1.5, np.zeros(3), m, np.zeros(3), n, 0.5, C, m, F64)
    i, j = np.meshgrid(np.arange(m), np.arange(n), indexing="ij")
    inside = (i >= j) if uplo == 1 else (i <= j)
    idx = (i + j * m)
    want = C.copy()
    want[idx[inside]] = 0.5 * C[idx[inside]]
    assert bits_equal(got, want)


def test_dgemmtr_quick_return(ctx):
    # alpha = 0 (or k = 0) with beta = 1: C comes back bit-identical
    n = 6
    C = orc.random_f64(n * n, -1, 1, 1030) * np.pi
    for alpha, k in ((0.0, n), (1.5, 0)):
        got = run_gemm(ctx, 1, 0, 0, n, n, k, alpha, orc.random_f64(n * max(k, 1), -1, 1, 1), n,
                       orc.random_f64(max(k, 1) * n, -1, 1, 2), max(k, 1), 1.0, C, n, F64)
        assert bits_equal(got, C)


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("n", [7, 150])
def test_dgemmtr_beta0_ignores_nan_inf_in_c(ctx, uplo, n):
    # test.dgemmtr.js:518-576: beta = 0 ignores NaN/Inf inside C's triangle;
    # the other triangle keeps its NaN
    A = orc.random_f64(n * n, -1, 1, 1)
    B = orc.random_f64(n * n, -1, 1, 2)
    C = orc.random_f64(n * n, -1, 1, 3)
    C[2 + 2 * n] = np.nan
    C[0 + (n - 1) * n] = np.nan      # (0, n-1): upper
    C[(n - 1) + 0 * n] = np.inf      # (n-1, 0): lower
    got = run_gemm(ctx, uplo, 0, 0, n, n, n, 1.5, A, n, B, n, 0.0, C, n, F64)
    i, j = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
    inside = ((i >= j) if uplo == 1 else (i <= j)).reshape(-1, order="F")
    assert np.all(np.isfinite(got[inside]))
    assert bits_equal(got[~inside], C[~inside])


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("beta", [0.0, 0.5])
def test_dgemmtr_alpha0_reads_neither_a_nor_b(ctx, uplo, beta):
    # test.dgemmtr.js:671-719
    n = 150
    A = orc.random_f64(n * n, -1, 1, 1)
    B = orc.random_f64(n * n, -1, 1, 2)
    A[1 + 2 * n], A[3] = np.nan, -np.inf
    B[2 + 3 * n] = np.inf
    C = orc.random_f64(n * n, -1, 1, 3)
    if beta == 0.0:
        C[4 + 4 * n] = np.nan
    got = run_gemm(ctx, uplo, 0, 0, n, n, n, 0.0, A, n, B, n, beta, C, n, F64)
    i, j = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
    inside = ((i >= j) if uplo == 1 else (i <= j)).reshape(-1, order="F")
    want = np.where(inside, 0.0 if beta == 0.0 else beta * C, C)  # beta = 0 writes +0
    assert bits_equal(got, want)


@pytest.mark.parametrize("n", [150, 400])
@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("trans", [0, 1])
def test_dsyrk_multi_tile(ctx, n, uplo, trans):
    # test.dsyrk.js:182-251: K = 9
    k = 9
    check_case(ctx, uplo, trans, 0, n, n, k, 1.5, 0.5, lda=(k if trans else n), ldb=0, ldc=n,
               dtype=F64, syrk=True)


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("trans", [0, 1])
def test_dsyrk_large_tier_and_padding(ctx, uplo, trans):
    n, k = 2100, 333
    check_case(ctx, uplo, trans, 0, n, n, k, 1.0, 0.75, lda=(k if trans else n) + 2, ldb=0,
               ldc=n + 3, dtype=F64, syrk=True)


def test_dsyrk_exact_on_integers(ctx):
    # test.dsyrk.js:342-390: small-integer inputs give exact results
    n, k = 33, 17
    rng = np.random.default_rng(7)
    A = rng.integers(-4, 5, size=n * k).astype(F64)
    C = rng.integers(-4, 5, size=n * n).astype(F64)
    got = run_gemm(ctx, 1, 0, 0, n, n, k, 2.0, A, n, None, n, -1.0, C, n, F64, syrk=True)
    Am = A.reshape(k, n).T
    i, j = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
    full = 2.0 * (Am @ Am.T) - C.reshape(n, n).T
    want = np.where(i >= j, full, C.reshape(n, n).T).T.reshape(-1)
    assert np.array_equal(got, want)
    keep = untouched_mask(n, n, n, n, 1)
    assert bits_equal(got[keep], C[keep])
