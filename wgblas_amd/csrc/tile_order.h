// Tile orders of the GEMM launches: which tile of C a workgroup computes.
//
// Included by gemm.hip (device code) and compiled for the host by the CPU
// test tests/test_tile_order.py, which defines the HIP function qualifiers
// away and checks that every order enumerates its tiles exactly once.
#pragma once

#include <stdint.h>

namespace wgb_tiles {

// Tile rows per band: consecutive logical tiles walk a band of kGroupM tile
// rows column by column, so the tiles an XCD runs at once (about 64) cover a
// kGroupM x 8 block of C and share kGroupM A panels and ~8 B panels.
constexpr int kGroupM = 8;
// MI355X's XCD count: the hardware deals workgroups round-robin over them.
constexpr int kXcds = 8;
// Tile rows per band of a triangle launch. Measured on ssyrk n = 8192,
// k = 4096 (HBM bytes per launch from FETCH_SIZE / WRITE_SIZE, against the
// 402.7 MB algorithmic): bands of 4 rows 2.75 GB (6.8x), 8 rows 2.86 GB
// (7.1x), 16 rows 3.49 GB (8.7x), at 142.0 / 142.0 / 141.1 TFLOP/s. A band's
// row panels stay hot for all of its columns, and each column panel is
// shared by the band's few consecutive tiles, which start close together.
constexpr int kGroupTri = 4;

// Number of tiles of a rows x cols tile grid that meet the lower (tile row
// >= tile col) triangle: row r holds min(r + 1, cols) tiles. The upper
// triangle of a grid is the lower triangle of its transpose.
__host__ __device__ inline int64_t triangle_tiles(int64_t rows, int64_t cols) {
  const int64_t full = rows < cols ? rows : cols;
  int64_t t = full * (full + 1) / 2;
  if (rows > cols) t += (rows - cols) * cols;
  return t;
}

// XCD-aware remap of workgroup w of a grid of n: give each XCD (w % kXcds)
// a contiguous run of logical tiles, so its L2 sees shared A and B panels.
__host__ __device__ inline int xcd_remap(int w, int n) {
  const int x = w % kXcds, j = w / kXcds;
  const int q = n / kXcds, r = n % kXcds;
  return x * q + (x < r ? x : r) + j;
}

// Lower-triangle tile L of a rows x cols tile grid, in bands of kGroupTri
// tile rows: band b holds rows [kGroupTri b, kGroupTri b + kGroupTri), walked column by
// column (column c of the band holds its rows r >= c). Every tile of the
// triangle gets exactly one L in [0, triangle_tiles(rows, cols)).
__host__ __device__ inline void triangle_decode_banded(int L, int rows, int cols, int &r, int &c) {
  // tiles in rows [0, x): sum over r < x of min(r + 1, cols)
  auto before = [cols](int64_t x) -> int64_t {
    if (x <= cols) return x * (x + 1) / 2;
    return (int64_t)cols * (cols + 1) / 2 + (x - cols) * cols;
  };
  // largest band b with before(kGroupTri b) <= L
  int lo = 0, hi = (rows + kGroupTri - 1) / kGroupTri - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (before((int64_t)mid * kGroupTri) <= (int64_t)L)
      lo = mid;
    else
      hi = mid - 1;
  }
  const int b0 = lo * kGroupTri;
  const int gh = rows - b0 < kGroupTri ? rows - b0 : kGroupTri;
  int o = (int)((int64_t)L - before(b0));
  // columns 0 .. min(b0, cols - 1) hold all gh rows of the band
  const int nfull = b0 + 1 < cols ? b0 + 1 : cols;
  if (o < nfull * gh) {
    c = o / gh;
    r = b0 + o % gh;
    return;
  }
  // then column c = b0 + 1 + j holds rows c .. b0 + gh - 1
  o -= nfull * gh;
  int cc = b0 + 1, cnt = gh - 1;
  while (o >= cnt) {
    o -= cnt;
    ++cc;
    --cnt;
  }
  c = cc;
  r = cc + o;
}

// Logical tile L -> (tile row tm, tile col tn) of a tiles_m x tiles_n grid.
// uplo 0 (full C): groups of kGroupM tile rows walked column by column.
// uplo 1 (lower, tm >= tn) / 2 (upper, tm <= tn): the banded triangle order
// (upper as the lower triangle of the transposed grid, i.e. bands of
// kGroupTri tile columns walked row by row).
__host__ __device__ inline void logical_tile(int L, int tiles_m, int tiles_n, int uplo, int &tm,
                                             int &tn) {
  if (uplo == 1) {
    triangle_decode_banded(L, tiles_m, tiles_n, tm, tn);
  } else if (uplo == 2) {
    triangle_decode_banded(L, tiles_n, tiles_m, tn, tm);
  } else {
    const int group_size = kGroupM * tiles_n;
    const int gid = L / group_size;
    const int first_m = gid * kGroupM;
    const int gm = tiles_m - first_m < kGroupM ? tiles_m - first_m : kGroupM;
    const int in_group = L % group_size;
    tm = first_m + in_group % gm;
    tn = in_group / gm;
  }
}

}  // namespace wgb_tiles
