"""GPU parity of the split-k tail of the GEMM launch.

When a launch's whole tiles fill at least one round of the chip's slots and
its last round would be at most half full (k at least 32 k-tiles), those
tail tiles are computed as k-slices (whole tiles first, then the slices) and
a fixup kernel adds the slices in split order. On an MI355X (256 CUs, two
resident 128-tiles per CU, 512 slots) the shapes below put a tail next to a
round of whole tiles on that path (3072 x 4096: 768 tiles, the last 256 in 2
slices each; 2944^2: 529 tiles, the last 17 in 16), for every operand
layout, the triangle routines and fp64. Results are checked by sampled rows
and columns against a float64 product under the reference's forward-error
bound plus a Freivalds projection over all of C, and whatever the call must
not touch (ld padding, the other triangle) is bit-checked.
"""
import pytest

from tests.helpers import run_gemm_props_case as run_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_split_tail_two_slices(ctx, ta, tb):
    # 24 x 32 = 768 tiles on 512 slots: 512 whole, the last 256 in 2 k-slices
    run_case(ctx, "sgemm", 0, ta, tb, 3072, 4096, 1024, 1.5, 0.5)


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
def test_sgemm_split_edges_and_k_tail(ctx, ta, tb):
    # 24 x 25 = 600 tiles: 512 whole, 88 in 5 slices; partial edge tiles and
    # k = 1777 (a partial last k-tile inside a slice)
    run_case(ctx, "sgemm", 0, ta, tb, 3071, 3073, 1777, -0.75, 1.0, ldc_pad=1, seed=12)


@pytest.mark.parametrize("ta,tb", [(0, 1), (1, 0)])
def test_sgemm_whole_tiles_plus_split_tail(ctx, ta, tb):
    # 23 x 23 = 529 tiles: 512 whole, the last 17 in 16 k-slices each
    run_case(ctx, "sgemm", 0, ta, tb, 2944, 2944, 2048, 1.0, 0.25, seed=13)


@pytest.mark.parametrize("uplo", [1, 2])
def test_sgemmtr_split(ctx, uplo):
    # 33 tile-rows: 561 triangle tiles, the last 49 in 8 slices
    run_case(ctx, "sgemmtr", uplo, 0, 1, 4200, 4200, 1024, 1.25, 0.5, seed=14)


@pytest.mark.parametrize("uplo", [1, 2])
@pytest.mark.parametrize("trans", [0, 1])
def test_ssyrk_split(ctx, uplo, trans):
    run_case(ctx, "ssyrk", uplo, trans, 0, 4200, 4200, 1000, 1.0, 0.75, seed=15)


@pytest.mark.parametrize("ta", [0, 1])
def test_dgemm_split(ctx, ta):
    # fp64: 576 tiles, the last 64 in 8 slices; transA takes the element-wise
    # partial store
    run_case(ctx, "dgemm", 0, ta, 1, 3072, 3072, 512, 1.0, 1.0, seed=16)
