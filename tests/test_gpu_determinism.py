"""Repeatability: the same call on the same inputs returns the same bits.

Every cross-block combination in the library has a fixed order: split-k
partial tiles are added in split order (split_fixup), the small-GEMM kernel
adds its waves' partial tiles in wave order, sgemv folds its splits in
order, and the reductions combine block partials in a fixed tree. This runs
each such path twice from identical inputs (fresh uploads of the same host
arrays) and requires bit-identical results, on shapes chosen to take those
paths: 512^3 (one-launch small kernel), 3000 x 3000 x 2000 and the ssyrk
case (a split-k tail on the 128 tier), dgemm with a split tail, sgemv N / T
with split contractions.
"""
import numpy as np
import pytest

from oracle import orc

pytestmark = pytest.mark.gpu


def twice(ctx, run, C):
    outs = []
    for _ in range(2):
        dC = ctx.upload(np.ascontiguousarray(C))
        run(dC)
        outs.append(dC.to_host())
        dC.free()
    return outs


@pytest.mark.parametrize("shape,ta,tb", [((512, 512, 512), 0, 0), ((3000, 3000, 2000), 1, 0),
                                         ((3000, 3000, 2000), 0, 1), ((777, 1500, 3001), 1, 1)])
def test_sgemm_repeats_bit_identical(ctx, shape, ta, tb):
    m, n, k = shape
    lda, ldb = (k if ta else m), (n if tb else k)
    A = orc.random_f32(lda * (m if ta else k), -1, 1, 1)
    B = orc.random_f32(ldb * (k if tb else n), -1, 1, 2)
    C = orc.random_f32(m * n, -1, 1, 3)
    dA, dB = ctx.upload(A), ctx.upload(B)
    a, b = twice(ctx, lambda dC: ctx.sgemm(ta, tb, m, n, k, 1.25, dA, lda, dB, ldb, 0.5, dC, m), C)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    dA.free()
    dB.free()


def test_ssyrk_split_tail_repeats_bit_identical(ctx):
    n, k = 3000, 2500
    A = orc.random_f32(n * k, -1, 1, 4)
    C = orc.random_f32(n * n, -1, 1, 5)
    dA = ctx.upload(A)
    a, b = twice(ctx, lambda dC: ctx.ssyrk(1, 0, n, k, 1.0, dA, n, 0.25, dC, n), C)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    dA.free()


def test_dgemm_repeats_bit_identical(ctx):
    m, n, k = 1500, 1400, 1300
    A = orc.random_f64(m * k, -1, 1, 6)
    B = orc.random_f64(n * k, -1, 1, 7)
    C = orc.random_f64(m * n, -1, 1, 8)
    dA, dB = ctx.upload(A), ctx.upload(B)
    a, b = twice(ctx, lambda dC: ctx.dgemm(0, 1, m, n, k, 1.0, dA, m, dB, n, 1.0, dC, m), C)
    assert np.array_equal(a.view(np.uint64), b.view(np.uint64))
    dA.free()
    dB.free()


@pytest.mark.parametrize("trans", [0, 1])
@pytest.mark.parametrize("m,n", [(4096, 6000), (8192, 3000)])
def test_sgemv_split_fold_repeats_bit_identical(ctx, trans, m, n):
    # 4096 rows: the transpose form's short-column kernel (4 columns per
    # wave); 8192 rows: its 8-column kernel; both split and fold
    A = orc.random_f32(m * n, -1, 1, 9)
    x = orc.random_f32(m if trans else n, -1, 1, 10)
    y = orc.random_f32(n if trans else m, -1, 1, 11)
    dA, dx = ctx.upload(A), ctx.upload(x)
    a, b = twice(ctx, lambda dy: ctx.sgemv(trans, m, n, 0.75, dA, m, dx, 1, 0.5, dy, 1), y)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    dA.free()
    dx.free()
