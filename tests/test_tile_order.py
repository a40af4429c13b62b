"""The GEMM launches' tile orders (wgblas_amd/csrc/tile_order.h), compiled
for the host with g++ from the same source the kernels include.

Every order must hand each tile of its part of C to exactly one logical
index (a missing tile leaves C unwritten, a repeated one races), inside the
requested triangle for sgemmtr / ssyrk (the other triangle is never touched,
as wgblas requires: src/shaders/sgemm_large.wgsl:78-83, 293-297). The banded
triangle order exists so that the ~64 tiles an XCD runs at once share A and B
panels; a window of 64 consecutive tiles must touch far fewer panels than the
~65 of a row-major walk over the triangle.
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "native", "tile_order_check.cc")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = str(tmp_path_factory.mktemp("tiles") / "tile_order_check")
    subprocess.run([gxx, "-O1", "-std=c++17", SRC, "-o", exe], check=True)

    def run(cases):
        inp = "".join(f"{r} {c} {u} {w}\n" for r, c, u, w in cases)
        out = subprocess.run([exe], input=inp, capture_output=True, text=True, check=True).stdout
        rows = [ln.split() for ln in out.splitlines() if not ln.startswith(" ")]
        assert len(rows) == len(cases), out
        return rows, out

    return run


def test_every_order_is_a_bijection(checker):
    cases = []
    for r in list(range(1, 20)) + [31, 32, 33, 63, 64, 65, 100, 129]:
        for c in [1, 2, 3, 7, 8, 9, 16, 17, 31, 64, 65, 130]:
            for u in (0, 1, 2):
                cases.append((r, c, u, 16))
    rows, out = checker(cases)
    bad = [x for x in rows if x[4] != "ok"]
    assert not bad, out


def test_triangle_count_matches_launch(checker):
    # the count the host launches (triangle_tiles) is what the decode covers
    rows, _ = checker([(64, 64, 1, 64), (64, 64, 2, 64), (65, 2, 1, 4), (2, 65, 2, 4)])
    assert [int(x[3]) for x in rows] == [2080, 2080, 2 * 3 // 2 + 63 * 2, 2 * 3 // 2 + 63 * 2]


def test_banded_triangle_shares_panels(checker):
    # config 5's launch: n = 8192 in 128-tiles, 64 x 64 grid, 2080 triangle
    # tiles; ~64 tiles resident per XCD (32 CUs x 2 blocks)
    rows, out = checker([(64, 64, 1, 64), (64, 64, 2, 64), (64, 64, 0, 64)])
    lower, upper, full = (int(x[5]) for x in rows)
    # triangle bands of kGroupTri = 4 rows and ~16 columns, full launches
    # kGroupM = 8 rows and ~8 columns, plus a spill into the next band
    assert lower <= 32 and upper <= 32, out
    assert full <= 32, out
