"""Parity at the full sizes of the benchmark configurations (wgblas's
benchmarks/*/wgblas/*.js: sgemm 512^3, sgemm 8192^3 in all four layouts,
the ragged 8191 x 8193 x 4097 case, dgemm 4096^3 in all four layouts, ten chained ssyrk calls at
8192 x 4096; the reductions' full sizes are in test_gpu_level1.py).

The inputs are the seeded device-generated ones bench.py times (their
generator is pinned bit-for-bit to the oracle in test_gpu_level1.py). At
these sizes the result is checked by properties that do not need a full
CPU GEMM:
  * sampled rows and columns of C (tile edges plus random ones) against an
    exact float64 computation under the reference's forward-error bound;
  * a Freivalds projection over ALL of C: C x against alpha op(A)(op(B) x) +
    beta C0 x for random +-1 vectors x, within the bound summed along rows
    (sum_j bound_ij |x_j|), which any wrong element beyond its bound breaks;
  * bit equality of everything the call must not touch (the other triangle
    for ssyrk, the ld padding).
"""
import numpy as np
import pytest

from oracle import orc
from tests.helpers import EPS32, EPS_DD, bits_equal, check_gemm_props, cm_view, op

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_config3_sgemm_8192(ctx, ta, tb):
    n = 8192
    buf = ctx.empty(3 * n * n, np.float32)
    ctx.fill_uniform(buf, -1.0, 1.0, 2)
    host = buf.to_host()
    A, B, C0 = host[:n * n], host[n * n:2 * n * n], host[2 * n * n:]
    ctx.sgemm(ta, tb, n, n, n, 1.5, buf.offset(0), n, buf.offset(n * n), n, 0.5,
              buf.offset(2 * n * n), n)
    C = buf.to_host()[2 * n * n:]
    buf.free()
    Am, Bm = cm_view(A, n, n, n), cm_view(B, n, n, n)
    check_gemm_props(cm_view(C, n, n, n), cm_view(C0, n, n, n), op(Am, ta), op(Bm, tb), 1.5, 0.5,
                     n, rows=(127, 128, 4095, 4096), cols=(127, 128, 4095, 4096), seed=ta * 2 + tb)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_config3_sgemm_ragged_ld(ctx, ta, tb):
    m, n, k = 8191, 8193, 4097
    ld = lambda r: ((r + 63) // 64) * 64 + 1
    a_rows, a_cols = (k, m) if ta else (m, k)
    b_rows, b_cols = (n, k) if tb else (k, n)
    lda, ldb, ldc = ld(a_rows), ld(b_rows), ld(m)
    sa, sb, sc = lda * a_cols, ldb * b_cols, ldc * n
    buf = ctx.empty(sa + sb + sc, np.float32)
    ctx.fill_uniform(buf, -1.0, 1.0, 2)
    host = buf.to_host()
    ctx.sgemm(ta, tb, m, n, k, 1.5, buf.offset(0), lda, buf.offset(sa), ldb, 0.5,
              buf.offset(sa + sb), ldc)
    out = buf.to_host()
    buf.free()
    A, B = host[:sa], host[sa:sa + sb]
    C0, C = host[sa + sb:], out[sa + sb:]
    # padding rows m..ldc-1 of every column are untouched
    pad = np.ones(sc, bool)
    pad[(np.arange(m)[:, None] + np.arange(n)[None, :] * ldc).reshape(-1)] = False
    assert bits_equal(C[pad], C0[pad])
    check_gemm_props(cm_view(C, m, n, ldc), cm_view(C0, m, n, ldc),
                     op(cm_view(A, a_rows, a_cols, lda), ta), op(cm_view(B, b_rows, b_cols, ldb), tb),
                     1.5, 0.5, k, rows=(127, 128, 8063, 8064, 8190), cols=(127, 128, 8192), seed=7)


@pytest.mark.parametrize("ta,tb", [(0, 1), (0, 0), (1, 0), (1, 1)])
def test_config4_dgemm_4096(ctx, ta, tb):
    # (0, 1) is config 4 itself; the other layouts run their own kernels
    n = 4096
    buf = ctx.empty(3 * n * n, np.float64)
    ctx.fill_uniform(buf, -1.0, 1.0, 3)
    host = buf.to_host()
    ctx.dgemm(ta, tb, n, n, n, 1.0, buf.offset(0), n, buf.offset(n * n), n, 1.0, buf.offset(2 * n * n), n)
    C = buf.to_host()[2 * n * n:]
    buf.free()
    A, B, C0 = host[:n * n], host[n * n:2 * n * n], host[2 * n * n:]
    check_gemm_props(cm_view(C, n, n, n), cm_view(C0, n, n, n), op(cm_view(A, n, n, n), ta),
                     op(cm_view(B, n, n, n), tb), 1.0, 1.0, n, eps=EPS_DD, kterm=2, cterm=3.0,
                     rows=(127, 128, 2047, 2048), cols=(127, 128, 2047, 2048), seed=3 + 4 * ta + 2 * tb)


def test_config5_ssyrk_chained(ctx):
    """uplo lower, n = 8192, k = 4096, A normal(0,1) seed 4, C uniform seed 5,
    alpha 1, beta 0.25, 10 chained resident calls; upper triangle bit-checked."""
    n, k = 8192, 4096
    dA = ctx.empty(n * k, np.float32)
    ctx.fill_normal(dA, 4)
    dC = ctx.empty(n * n, np.float32)
    ctx.fill_uniform(dC, -1.0, 1.0, 5)
    A = dA.to_host()
    C0 = dC.to_host()
    ctx.ssyrk(1, 0, n, k, 1.0, dA, n, 0.25, dC, n)
    C1 = dC.to_host()
    Am = cm_view(A, n, k, n)
    check_gemm_props(cm_view(C1, n, n, n), cm_view(C0, n, n, n), Am, Am.T, 1.0, 0.25, k,
                     rows=(127, 128, 4095, 4096, 8191), cols=(0, 127, 128, 4096), seed=5, uplo=1)
    for _ in range(9):
        ctx.ssyrk(1, 0, n, k, 1.0, dA, n, 0.25, dC, n)
    C10 = dC.to_host()
    upper = np.triu(np.ones((n, n), bool), 1).T.reshape(-1)  # column-major strictly upper
    assert bits_equal(C10[upper], C0[upper])
    # closed form after 10 calls: (1 + b + ... + b^9) A A^T + b^10 C0, on sampled rows
    b = 0.25
    geo = sum(b ** t for t in range(10))
    rows = [0, 1, 128, 4096, 8191]
    A64 = np.asarray(Am, np.float64)
    exact = geo * (A64[rows, :] @ A64.T) + b ** 10 * np.asarray(cm_view(C0, n, n, n)[rows, :], np.float64)
    got = np.asarray(cm_view(C10, n, n, n)[rows, :], np.float64)
    absd = np.abs(A64[rows, :]) @ np.abs(A64.T)
    mask = np.arange(n)[None, :] <= np.array(rows)[:, None]
    bound = 10 * EPS32 * ((k + 1) * geo * absd + 1.0)
    assert np.all(np.where(mask, np.abs(got - exact) <= bound, True))
    dA.free()
    dC.free()


def test_config1_sgemm_512_full_oracle(ctx):
    # A then B from one seed-0 stream, C zero: the inputs bench.py times
    n = 512
    AB = orc.random_f32(2 * n * n, -1, 1, 0)
    A, B = AB[:n * n], AB[n * n:]
    C0 = np.zeros(n * n, np.float32)
    dA, dB, dC = ctx.upload(A), ctx.upload(B), ctx.upload(C0)
    ctx.sgemm(0, 0, n, n, n, 1.0, dA, n, dB, n, 0.0, dC, n)
    got = dC.to_host()
    ref, absdot = orc.gemm_ld(0, 0, 0, n, n, n, 1.0, A.astype(np.float64), n, B.astype(np.float64),
                              n, 0.0, C0.astype(np.float64), n)
    bound = EPS32 * (n + 1) * absdot
    assert np.all(np.abs(got - ref) <= bound)
