"""GPU parity of GEMM edge tiles (tiles that cross m or n).

Edge tiles stream their whole k-tiles with clamped addresses: a lane whose
rows lie past m (or n) reads a row of the matrix that is in range, and an
mn-contiguous vector that is only partly in range reads into the next
column; those values reach only C rows / columns that are never written. The
last whole k-tile and a partial k-tile take element guards (their address
bounds are modelled on the CPU in test_gemm_edge_model.py). These shapes
cover both tiers, every operand layout, ld padding, leading dimensions of 1-3
(vectors that overrun their column), triangles and fp64; each result is
checked by sampled rows and columns under the forward-error bound, a
Freivalds projection and bit checks of what must stay untouched.
"""
import pytest

from tests.helpers import run_gemm_props_case as run_case

pytestmark = pytest.mark.gpu

LAYOUTS = [(0, 0), (0, 1), (1, 0), (1, 1)]


@pytest.mark.parametrize("ta,tb", LAYOUTS)
@pytest.mark.parametrize("shape", [(130, 250, 300), (1000, 1001, 999), (2100, 2050, 700)])
def test_sgemm_edge_tiles(ctx, ta, tb, shape):
    m, n, k = shape
    run_case(ctx, "sgemm", 0, ta, tb, m, n, k, 1.5, 0.5, seed=21)


@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_sgemm_edge_tiles_padded_ld(ctx, ta, tb):
    run_case(ctx, "sgemm", 0, ta, tb, 777, 555, 333, -1.0, 0.25, seed=22, lda_pad=5, ldb_pad=3,
             ldc_pad=7)


@pytest.mark.parametrize("shape,ta,tb", [
    ((2, 300, 500), 0, 0),    # A mn-contiguous with lda = 2
    ((3, 300, 500), 0, 1),    # lda = 3
    ((300, 3, 500), 0, 1),    # B transposed, ldb = 3
    ((300, 2, 500), 1, 1),    # B transposed, ldb = 2
    ((1, 1, 600), 0, 0),      # every vector overruns its column
])
def test_sgemm_thin_edges(ctx, shape, ta, tb):
    m, n, k = shape
    run_case(ctx, "sgemm", 0, ta, tb, m, n, k, 1.0, 1.0, seed=23, ldc_pad=0)


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("ta,tb", [(0, 1), (1, 0)])
def test_sgemmtr_edge_tiles(ctx, uplo, ta, tb):
    run_case(ctx, "sgemmtr", uplo, ta, tb, 1111, 1111, 400, 1.25, 0.5, seed=24)


@pytest.mark.parametrize("trans", [0, 1])
def test_ssyrk_edge_tiles(ctx, trans):
    run_case(ctx, "ssyrk", 1, trans, 0, 2100, 2100, 300, 1.0, 0.75, seed=25)


@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_dgemm_edge_tiles(ctx, ta, tb):
    run_case(ctx, "dgemm", 0, ta, tb, 700, 650, 333, 1.0, 1.0, seed=26)
