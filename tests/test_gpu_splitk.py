"""GPU parity of the split-k tail of the GEMM launch.

When a launch's last round of tiles would be at most half full, those tail
tiles are computed as k-slices (whole tiles first, then the slices) and a
fixup kernel adds the slices in split order. On an MI355X (256 CUs, two
resident 128-tiles per CU) the shapes below put all tiles (256-tile grids),
or a few tail tiles next to many whole ones (2944^2: 529 tiles), on that path,
for every operand layout, the triangle routines and fp64. Results are checked
by sampled rows and columns against a float64 product under the reference's
forward-error bound plus a Freivalds projection over all of C, and whatever
the call must not touch (ld padding, the other triangle) is bit-checked.
"""
import numpy as np
import pytest

from tests.helpers import EPS_DD, bits_equal, check_gemm_props, cm_view, op, untouched_mask

pytestmark = pytest.mark.gpu


def run_case(ctx, kind, uplo, ta, tb, m, n, k, alpha, beta, ldc_pad=3, seed=11):
    dt = np.float64 if kind == "dgemm" else np.float32
    a_rows, a_cols = (k, m) if ta else (m, k)
    if kind == "ssyrk":
        tb = 1 - ta
        b_rows, b_cols = a_rows, a_cols
    else:
        b_rows, b_cols = (n, k) if tb else (k, n)
    lda, ldb, ldc = a_rows, b_rows, m + ldc_pad
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
    edges = (0, 127, 128, 255, 256, min(m, n) - 1)
    kw = dict(eps=EPS_DD, kterm=2, cterm=3.0) if kind == "dgemm" else {}
    check_gemm_props(cm_view(C, m, n, ldc), cm_view(C0, m, n, ldc), Am, Bm, alpha, beta, k,
                     rows=edges, cols=edges, seed=seed, uplo=uplo, **kw)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_all_tiles_split(ctx, ta, tb):
    # 16 x 16 = 256 tiles on 512 slots: every tile in 2 k-slices
    run_case(ctx, "sgemm", 0, ta, tb, 2048, 2048, 1024, 1.5, 0.5)


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
def test_sgemm_split_edges_and_k_tail(ctx, ta, tb):
    # partial edge tiles and k = 777 (a partial last k-tile inside a slice)
    run_case(ctx, "sgemm", 0, ta, tb, 1999, 2001, 777, -0.75, 1.0, ldc_pad=1, seed=12)


@pytest.mark.parametrize("ta,tb", [(0, 1), (1, 0)])
def test_sgemm_whole_tiles_plus_split_tail(ctx, ta, tb):
    # 23 x 23 = 529 tiles: 512 whole, the last 17 in 16 k-slices each
    run_case(ctx, "sgemm", 0, ta, tb, 2944, 2944, 2048, 1.0, 0.25, seed=13)


@pytest.mark.parametrize("uplo", [1, 2])
def test_sgemmtr_split(ctx, uplo):
    # 22 tile-rows: 253 triangle tiles, all split
    run_case(ctx, "sgemmtr", uplo, 0, 1, 2800, 2800, 300, 1.25, 0.5, seed=14)


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("trans", [0, 1])
def test_ssyrk_split(ctx, uplo, trans):
    run_case(ctx, "ssyrk", uplo, trans, 0, 2800, 2800, 1000, 1.0, 0.75, seed=15)


@pytest.mark.parametrize("ta", [0, 1])
def test_dgemm_split(ctx, ta):
    # fp64: 256 tiles split in 2; transA takes the element-wise partial store
    run_case(ctx, "dgemm", 0, ta, 1, 2048, 2048, 512, 1.0, 1.0, seed=16)
