// Host build of wgblas_amd/csrc/tile_order.h (the GEMM launches' tile
// orders) for tests/test_tile_order.py. For each grid given on stdin as
// "rows cols uplo window" it checks that logical tiles 0..count-1 decode to
// distinct in-range tiles of the requested part of C (all of it, the lower
// or the upper triangle), that xcd_remap permutes 0..count-1, and prints the
// largest number of distinct A panels (tile rows) plus B panels (tile
// columns) that `window` consecutive logical tiles of one XCD's run touch.
#define __host__
#define __device__
#include <cstdio>
#include <set>
#include <vector>

#include "../../wgblas_amd/csrc/tile_order.h"

using namespace wgb_tiles;

int main() {
  int rows, cols, uplo, window;
  while (std::scanf("%d %d %d %d", &rows, &cols, &uplo, &window) == 4) {
    long long count = uplo == 1   ? triangle_tiles(rows, cols)
                      : uplo == 2 ? triangle_tiles(cols, rows)
                                  : (long long)rows * cols;
    std::vector<char> seen((size_t)rows * cols, 0);
    std::vector<int> tr(count), tc(count);
    const char *err = nullptr;
    for (long long L = 0; L < count && !err; ++L) {
      int r = -1, c = -1;
      logical_tile((int)L, rows, cols, uplo, r, c);
      tr[L] = r;
      tc[L] = c;
      if (r < 0 || r >= rows || c < 0 || c >= cols) err = "out of range";
      else if (uplo == 1 && r < c) err = "above the diagonal";
      else if (uplo == 2 && r > c) err = "below the diagonal";
      else if (seen[(size_t)r * cols + c]++) err = "tile decoded twice";
    }
    std::vector<char> hit(count, 0);
    for (long long w = 0; w < count && !err; ++w) {
      int L = xcd_remap((int)w, (int)count);
      if (L < 0 || L >= count || hit[L]++) err = "xcd_remap is not a permutation";
    }
    int worst = 0;
    if (!err) {
      // one XCD's contiguous run of logical tiles, windows of `window`
      for (long long s = 0; s + window <= count; s += window / 4 > 0 ? window / 4 : 1) {
        std::set<int> pr, pc;
        for (long long L = s; L < s + window; ++L) {
          pr.insert(tr[L]);
          pc.insert(tc[L]);
        }
        int t = (int)(pr.size() + pc.size());
        if (t > worst) worst = t;
      }
    }
    std::printf("%d %d %d %lld %s %d\n", rows, cols, uplo, count, err ? "FAIL" : "ok", worst);
    if (err) std::printf("  %s\n", err);
  }
  return 0;
}
