// sgemv (wgblas src/sgemv/sgemv.mjs:19-254, shaders sgemv_n.wgsl,
// sgemv_t.wgsl, reduce_partials.wgsl) and its native-fp64 form dgemv
// (src/dgemv/dgemv.mjs:23-341), column-major as in BLAS, and further down
// the rank-1 / rank-2 updates sger / dger, ssyr / dsyr, ssyr2 / dsyr2
// (src/{sger,dger,ssyr,dsyr,ssyr2,dsyr2}/*.mjs). gemv:
//   trans = N: y (m) <- alpha A x + beta y, x of length n;
//   trans = T: y (n) <- alpha A^T x + beta y, x of length m.
//
// Both forms read A once and are HBM-bound. A lane's loads are 4 consecutive
// elements (16 bytes in fp32, 32 in fp64).
//   N: a lane owns 4 consecutive rows in each of kGroupsN 1024-row groups
//      (one 4-element load per group and column, kStepN columns per step), and a
//      block walks a long run of columns (few, deep blocks); the
//      columns are walked in order and a column whose x entry is zero is
//      skipped, as reference BLAS does for this form (so 0 * Inf or 0 * NaN
//      in that column never reaches y).
//   T: a wave owns 8 columns (4 for short columns) and walks the rows 512
//      at a time (2 x 4 per lane, 4-element loads), keeping each x chunk in
//      registers for all of its columns;
//      the dot products are folded with wave shuffles. No zero skipping: the
//      dot-product form of reference BLAS takes every term.
// When the output alone gives too few blocks to stream HBM, the contraction
// dimension is split: each split writes partial sums, and a fold kernel adds
// the splits in order (deterministic) and applies alpha and beta.
#include "common.h"

#include <hip/hip_runtime.h>

#include "wgblas_hip.h"

namespace {

using wgb::fail;

constexpr int kThreads = 256;
// T form: columns per wave. 8 (x reused from registers for 8 columns);
// columns of at most kShortColsRows rows take 4, which gives twice the
// waves: measured on MI355X at 2048 x 65536, 4.8 -> 6.4 TB/s, while 4 was
// slower at 8192^2 (5.3 -> 4.8) and even at 16384^2 and 32768^2.
constexpr int kColsPerWave = 8;
constexpr int kColsPerWaveShort = 4;
constexpr int64_t kShortColsRows = 4096;
// N form: columns loaded per step, 1024-row groups per block, the blocks
// aimed for and the fewest columns per split. Measured on MI355X over
// 2048 x 65536, 8192^2, 16384^2, 32768^2 and 65536 x 2048 (sweep of 1 or 2
// groups, 256 / 512 / 1024 target blocks, 256 or 512 columns): one group,
// 8 columns per step, about 256 blocks of at least 256 columns each gave
// the best geometric mean, 5.92 TB/s against 5.06 for 4 groups x 4 columns
// with 2048 blocks of 64 columns (16384^2: 6.24 against 5.77 TB/s); fewer
// splits also mean fewer partial sums to write and fold.
constexpr int kStepN = 8;
constexpr int kGroupsN = 1;
constexpr int kTargetBlocksN = 256;
constexpr int kMinColsN = 256;
constexpr int kTargetBlocks = 2048;  // T form: blocks that keep HBM streaming

int64_t imax(int64_t a, int64_t b) { return a > b ? a : b; }
int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

template <typename T>
using vec4 = T __attribute__((ext_vector_type(4)));

// A is streamed once: non-temporal 4-element loads keep it from displacing x
// and the partial sums in the caches.
template <typename T>
__device__ __forceinline__ vec4<T> ld_nt(const T *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const vec4<T> *>(p));
}

// p aligned to 4 elements (the vector loads' alignment)
template <typename T>
bool aligned4(const T *p) {
  return ((uintptr_t)p % (4 * sizeof(T))) == 0;
}

// Writes one output element: alpha * acc + beta * y (beta == 0 never reads y).
template <typename T>
__device__ __forceinline__ void store_y(T *y, int64_t idx, T acc, T alpha, T beta) {
  T v = alpha * acc;
  if (beta != (T)0) v = fma(beta, y[idx], v);
  y[idx] = v;
}

// N form. Block b, split s: columns [s*cps, min(n, (s+1)*cps)); rows in
// kGroupsN groups of 1024, lane t of group g owning rows
// [b*1024*kGroupsN + g*1024 + 4t, +4) (every load instruction of a wave
// reads 256 elements of one column). VEC: lda % 4 == 0 and A aligned to 4
// elements.
template <typename T, bool VEC>
__global__ __launch_bounds__(kThreads) void gemv_n_kernel(int64_t m, int64_t n,
                                                          const T *__restrict__ A, int64_t lda,
                                                          const T *__restrict__ x, int64_t incx,
                                                          int64_t cps, T *__restrict__ part,
                                                          T alpha, T beta,
                                                          T *__restrict__ y, int64_t incy) {
  typedef vec4<T> f4;
  constexpr int G = kGroupsN;
  const int64_t rb = (int64_t)blockIdx.x * (4 * kThreads * G) + 4 * threadIdx.x;
  const int64_t j0 = (int64_t)blockIdx.y * cps;
  const int64_t j1 = j0 + cps < n ? j0 + cps : n;
  if (rb >= m) return;
  // rows past m read row m-1 (in bounds) and are never stored
  int64_t ir[G][4];
  bool full[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int64_t i0 = rb + (int64_t)g * 4 * kThreads;
    full[g] = i0 + 4 <= m;
#pragma unroll
    for (int q = 0; q < 4; ++q) ir[g][q] = i0 + q < m ? i0 + q : m - 1;
  }
  T acc[G][4];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[g][q] = (T)0;
  auto load = [&](const T *col, int g) -> f4 {
    if (VEC && full[g]) return ld_nt(col + ir[g][0]);
    return f4{col[ir[g][0]], col[ir[g][1]], col[ir[g][2]], col[ir[g][3]]};
  };
  int64_t j = j0;
  // kStepN columns per step, every load issued before the arithmetic
  for (; j + kStepN <= j1; j += kStepN) {
    T xv[kStepN];
    f4 av[kStepN][G];
#pragma unroll
    for (int c = 0; c < kStepN; ++c) xv[c] = x[(j + c) * incx];
#pragma unroll
    for (int c = 0; c < kStepN; ++c)
#pragma unroll
      for (int g = 0; g < G; ++g) av[c][g] = load(A + (j + c) * lda, g);
#pragma unroll
    for (int c = 0; c < kStepN; ++c) {
      if (xv[c] != (T)0) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[g][q] = fma(av[c][g][q], xv[c], acc[g][q]);
      }
    }
  }
  for (; j < j1; ++j) {
    const T xj = x[j * incx];
    f4 a[G];
#pragma unroll
    for (int g = 0; g < G; ++g) a[g] = load(A + j * lda, g);
    if (xj != (T)0) {
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[g][q] = fma(a[g][q], xj, acc[g][q]);
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int64_t i0 = rb + (int64_t)g * 4 * kThreads;
    const int rows = i0 >= m ? 0 : (full[g] ? 4 : (int)(m - i0));
    for (int q = 0; q < rows; ++q) {
      if (part)
        part[(int64_t)blockIdx.y * m + i0 + q] = acc[g][q];
      else
        store_y(y, (i0 + q) * incy, acc[g][q], alpha, beta);
    }
  }
}

// T form. Wave w (4 per block) owns columns [CPW w, CPW w + CPW) of split s, rows
// [s*rps, min(m, (s+1)*rps)). VEC: lda % 4 == 0, A 16-byte aligned, incx == 1
// and x 16-byte aligned (rps is a multiple of 4, so every 4-row group of a
// split starts aligned).
template <typename T, bool VEC, int CPW>
__global__ __launch_bounds__(kThreads) void gemv_t_kernel(int64_t m, int64_t n,
                                                          const T *__restrict__ A, int64_t lda,
                                                          const T *__restrict__ x, int64_t incx,
                                                          int64_t rps, T *__restrict__ part,
                                                          T alpha, T beta,
                                                          T *__restrict__ y, int64_t incy) {
  typedef vec4<T> f4;
  const int lane = threadIdx.x & 63;
  const int64_t col0 = ((int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)) * CPW;
  if (col0 >= n) return;  // wave-uniform
  const int64_t r0 = (int64_t)blockIdx.y * rps;
  const int64_t r1 = r0 + rps < m ? r0 + rps : m;
  // columns past n repeat column n-1 (in bounds) and are never stored
  const T *col[CPW];
#pragma unroll
  for (int c = 0; c < CPW; ++c) col[c] = A + (col0 + c < n ? col0 + c : n - 1) * lda;
  T acc[CPW];
#pragma unroll
  for (int c = 0; c < CPW; ++c) acc[c] = (T)0;
  int64_t i = r0 + 4 * lane;
  if (VEC) {
    // two 256-row groups per step: 16 loads of A in flight per lane
    for (; i + 256 + 4 <= r1; i += 512) {
      const f4 xv0 = *reinterpret_cast<const f4 *>(x + i);
      const f4 xv1 = *reinterpret_cast<const f4 *>(x + i + 256);
      f4 av0[CPW], av1[CPW];
#pragma unroll
      for (int c = 0; c < CPW; ++c) {
        av0[c] = ld_nt(col[c] + i);
        av1[c] = ld_nt(col[c] + i + 256);
      }
      // fp64: every load of the step is issued before the arithmetic. Left
      // to itself the scheduler placed each 16-byte load just before its
      // FMAs and waited for it (one load in flight: 16384^2 at 3.5 TB/s).
      if constexpr (sizeof(T) == 8) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < CPW; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[c] = fma(av0[c][q], xv0[q], acc[c]);
#pragma unroll
      for (int c = 0; c < CPW; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[c] = fma(av1[c][q], xv1[q], acc[c]);
    }
  }
  for (; i < r1; i += 256) {
    if (VEC && i + 4 <= r1) {
      const f4 xv = *reinterpret_cast<const f4 *>(x + i);
      f4 av[CPW];
#pragma unroll
      for (int c = 0; c < CPW; ++c) av[c] = ld_nt(col[c] + i);
#pragma unroll
      for (int c = 0; c < CPW; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[c] = fma(av[c][q], xv[q], acc[c]);
    } else {
      const int cnt = r1 - i < 4 ? (int)(r1 - i) : 4;
      for (int q = 0; q < cnt; ++q) {
        const T xv = x[(i + q) * incx];
#pragma unroll
        for (int c = 0; c < CPW; ++c) acc[c] = fma(col[c][i + q], xv, acc[c]);
      }
    }
  }
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc[c] += __shfl_xor(acc[c], off, 64);
  }
  if (lane < CPW && col0 + lane < n) {
    T v = acc[0];
#pragma unroll
    for (int c = 1; c < CPW; ++c) v = lane == c ? acc[c] : v;
    if (part)
      part[(int64_t)blockIdx.y * n + col0 + lane] = v;
    else
      store_y(y, (col0 + lane) * incy, v, alpha, beta);
  }
}

// One fold pass over groups of kFold splits: block (b, g) adds splits
// [g*kFold, min(splits, (g+1)*kFold)) of outputs [256 b, 256 b + 256) in
// split order, with all of a group's loads in flight (clamped addresses, so
// none is guarded). The last pass (one group) writes alpha * sum + beta * y;
// earlier ones write the group sums to out[g*len + i] for the next pass.
constexpr int kFold = 32;
template <typename T>
__global__ __launch_bounds__(kThreads) void gemv_fold_kernel(int64_t len, int64_t splits,
                                                             const T *__restrict__ part,
                                                             T *__restrict__ out, T alpha,
                                                             T beta, T *__restrict__ y,
                                                             int64_t incy) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= len) return;
  const int64_t s0 = (int64_t)blockIdx.y * kFold;
  const int64_t last = (s0 + kFold < splits ? s0 + kFold : splits) - 1;
  T v[kFold];
#pragma unroll
  for (int q = 0; q < kFold; ++q) v[q] = part[(s0 + q < last ? s0 + q : last) * len + i];
  T sum = v[0];
#pragma unroll
  for (int q = 1; q < kFold; ++q)
    if (s0 + q <= last) sum += v[q];
  if (gridDim.y == 1 && out == nullptr)
    store_y(y, i * incy, sum, alpha, beta);
  else
    out[(int64_t)blockIdx.y * len + i] = sum;
}

// y <- beta * y over len elements (0 when beta == 0): alpha == 0.
template <typename T>
__global__ __launch_bounds__(kThreads) void scale_y_kernel(int64_t len, T beta, T *y,
                                                           int64_t incy) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < len) y[i * incy] = beta == (T)0 ? (T)0 : beta * y[i * incy];
}

// Rank-1 and rank-2 updates, A m x n column-major:
//   ger  (UPLO 0, !TWO): A += alpha x y^T;
//   syr  (UPLO 1 / 2, !TWO, y = x): the lower (i >= j) / upper (i <= j)
//        triangle of A += alpha x x^T;
//   syr2 (UPLO 1 / 2, TWO): that triangle of A += alpha x y^T + alpha y x^T.
// Block (b, c): rows [1024 b, +1024) (4 consecutive rows per lane, its x
// (and y) entries held in registers), columns [c cpb, min(n, (c+1) cpb)),
// kStepG at a time with all of a step's A loads in flight. Column j takes
// t1 = alpha y[j] (and t2 = alpha x[j]) and A(i, j) = fma(x[i], t1, A(i, j))
// (then fma(y[i], t2, .)); a column whose y entry (for syr2: both entries)
// is zero is neither computed nor written, reference BLAS's skip: Infinity or
// NaN in the row vector never meets that zero. A is read and written once:
// HBM-bound, 2 m n elements of traffic (half that for a triangle).
constexpr int kStepG = 8;
template <typename T, bool VEC, int UPLO, bool TWO>
__global__ __launch_bounds__(kThreads) void rank_update_kernel(
    int64_t m, int64_t n, T alpha, const T *__restrict__ x, int64_t incx, const T *__restrict__ y,
    int64_t incy, T *__restrict__ A, int64_t lda, int64_t cpb) {
  typedef vec4<T> f4;
  const int64_t r0 = (int64_t)blockIdx.x * (4 * kThreads);
  const int64_t i0 = r0 + 4 * threadIdx.x;
  if (i0 >= m) return;
  const int rows = i0 + 4 <= m ? 4 : (int)(m - i0);
  f4 xv, yv;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    xv[q] = q < rows ? x[(i0 + q) * incx] : (T)0;
    yv[q] = TWO && q < rows ? y[(i0 + q) * incy] : (T)0;
  }
  int64_t j0 = (int64_t)blockIdx.y * cpb;
  int64_t j1 = j0 + cpb < n ? j0 + cpb : n;
  // triangle: the block's columns split into whole ones (every row of the
  // block inside the triangle) and diagonal ones (rows masked per element)
  const int64_t rlast = r0 + 4 * kThreads - 1;  // the block's last row
  int64_t d0 = j0, d1 = j0;                     // diagonal columns [d0, d1)
  if (UPLO == 1) {                              // lower: i >= j
    if (j1 > rlast + 1) j1 = rlast + 1;
    d0 = j0 > r0 + 1 ? j0 : r0 + 1;
    d1 = j1;
    if (d0 > d1) d0 = d1;
  } else if (UPLO == 2) {  // upper: i <= j
    if (j0 < r0) j0 = r0;
    d0 = j0;
    d1 = j1 < rlast ? j1 : rlast;
    if (d1 < d0) d1 = d0;
  }
  // update of one column's 4 rows (masked rows keep their value)
  auto column_scalars = [&](int64_t j, T &t1, T &t2) -> bool {
    const T c1 = y[j * incy];
    const T c2 = TWO ? x[j * incx] : (T)0;
    t1 = alpha * c1;
    t2 = alpha * c2;
    return c1 != (T)0 || (TWO && c2 != (T)0);
  };
  auto update = [&](f4 &a, T t1, T t2) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      a[q] = fma(xv[q], t1, a[q]);
      if (TWO) a[q] = fma(yv[q], t2, a[q]);
    }
  };
  // FULL: every row of the block inside m (a block-uniform choice): whole
  // non-temporal vectors with no per-lane branch between them, a step's
  // loads all issued together; otherwise element accesses with clamped rows.
  // (A per-lane choice between the two, measured for ger at 16384^2 with
  // 512 blocks on one box: fp32 5.0 against 5.5 TB/s.) MASK (the diagonal
  // columns of a triangle): the same loads and arithmetic, and each lane
  // stores only its rows inside the triangle (whole vectors where all four
  // are).
  auto walk = [&](auto full_tag, auto mask_tag, int64_t ja, int64_t jb) {
    constexpr bool FULL = decltype(full_tag)::value;
    constexpr bool MASK = decltype(mask_tag)::value;
    auto load = [&](const T *col) -> f4 {
      if constexpr (FULL) return ld_nt(col + i0);
      f4 v;
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = col[i0 + (q < rows ? q : 0)];
      return v;
    };
    auto store = [&](T *col, const f4 &v, int64_t j) {
      if constexpr (MASK) {
        const bool all = UPLO == 1 ? i0 >= j : i0 + rows - 1 <= j;
        if (!all) {
          for (int q = 0; q < rows; ++q) {
            const int64_t i = i0 + q;
            if (UPLO == 1 ? i >= j : i <= j) col[i] = v[q];
          }
          return;
        }
      }
      if constexpr (FULL) {
        __builtin_nontemporal_store(v, reinterpret_cast<f4 *>(col + i0));
      } else {
        for (int q = 0; q < rows; ++q) col[i0 + q] = v[q];
      }
    };
    int64_t j = ja;
    for (; j + kStepG <= jb; j += kStepG) {
      T t1[kStepG], t2[kStepG];
      bool live[kStepG];
      f4 a[kStepG];
#pragma unroll
      for (int c = 0; c < kStepG; ++c) live[c] = column_scalars(j + c, t1[c], t2[c]);
#pragma unroll
      for (int c = 0; c < kStepG; ++c) a[c] = load(A + (j + c) * lda);
#pragma unroll
      for (int c = 0; c < kStepG; ++c) {
        if (live[c]) {  // uniform: the column's entries
          update(a[c], t1[c], t2[c]);
          store(A + (j + c) * lda, a[c], j + c);
        }
      }
    }
    for (; j < jb; ++j) {
      T t1, t2;
      if (column_scalars(j, t1, t2)) {
        f4 a = load(A + j * lda);
        update(a, t1, t2);
        store(A + j * lda, a, j);
      }
    }
  };
  const bool whole_rows = VEC && rlast < m;
  auto walk_range = [&](auto mask_tag, int64_t ja, int64_t jb) {
    if (ja >= jb) return;
    if (whole_rows)
      walk(std::true_type{}, mask_tag, ja, jb);
    else
      walk(std::false_type{}, mask_tag, ja, jb);
  };
  if (UPLO == 0) {
    walk_range(std::false_type{}, j0, j1);
    return;
  }
  // whole columns, then the diagonal ones: row i of column j is stored
  // where i >= j (lower) or i <= j (upper)
  if (UPLO == 1)
    walk_range(std::false_type{}, j0, d0);
  else
    walk_range(std::false_type{}, d1, j1);
  walk_range(std::true_type{}, d0, d1);
}

// ger (uplo 0, y given), syr (uplo 1 / 2, y == x, !two), syr2 (uplo 1 / 2,
// two): argument checks, reference BLAS's quick returns (m or n zero, alpha
// zero: A untouched, vectors unread; src/sger/sger.mjs:86, 103,
// src/ssyr/ssyr.mjs:59, 75), one launch.
template <typename T>
int rank_update(wgb_ctx *ctx, int uplo, bool two, int64_t m, int64_t n, T alpha, const T *x,
                int64_t incx, const T *y, int64_t incy, T *A, int64_t lda) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if (uplo != 0 && uplo != WGB_LOWER && uplo != WGB_UPPER)
    return fail(WGB_ERR_INVALID_VALUE, "uplo must be WGB_LOWER or WGB_UPPER");
  if (m < 0 || n < 0) return fail(WGB_ERR_INVALID_VALUE, "m and n must be non-negative");
  if (lda < imax(1, m)) return fail(WGB_ERR_INVALID_VALUE, "lda must be >= max(1, rows of A)");
  if (incx <= 0 || incy <= 0) return fail(WGB_ERR_INVALID_VALUE, "incx and incy must be positive");
  if (m == 0 || n == 0 || alpha == (T)0) return WGB_OK;
  if (!A || !x || !y) return fail(WGB_ERR_INVALID_VALUE, "A, x or y is null");
  wgb::timing_begin(ctx);
  const int64_t bx = cdiv(m, 4 * kThreads);
  // column chunks: about one block per CU in all for ger (each a long run of
  // columns), at least kStepG columns each. Measured at 16384^2 on one box,
  // blocks in all against TB/s (fp32 / fp64): 128 3.5 / 3.7, 256 5.7 / 5.2,
  // 384 5.7 / 4.1, 512 5.5 / 4.9, 2048 4.8 / 4.7. A triangle's blocks do
  // work that varies with their row; for fp32, four times as many, shorter
  // blocks even it out (lower 16384, blocks per CU 1 / 2 / 4 / 8 / 16: ssyr
  // 2.4 / 3.4 / 3.5 / 3.6 / 3.3 TB/s), fp64 kept one per CU (dsyr 3.4 / 3.0 /
  // 3.1 / 3.1 / 3.2).
  const int64_t cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
  const int64_t target = uplo == 0 || sizeof(T) == 8 ? cus : 4 * cus;
  int64_t chunks = cdiv(target, bx);
  if (chunks > cdiv(n, kStepG)) chunks = cdiv(n, kStepG);
  if (chunks > 65535) chunks = 65535;
  if (chunks < 1) chunks = 1;
  const int64_t cpb = cdiv(n, chunks);
  const dim3 grid((unsigned)bx, (unsigned)cdiv(n, cpb));
  const bool vec = lda % 4 == 0 && aligned4(A);
  auto launch = [&](auto kern) {
    kern<<<grid, kThreads, 0, ctx->stream>>>(m, n, alpha, x, incx, y, incy, A, lda, cpb);
  };
  if (uplo == 0)
    launch(vec ? rank_update_kernel<T, true, 0, false> : rank_update_kernel<T, false, 0, false>);
  else if (uplo == WGB_LOWER && !two)
    launch(vec ? rank_update_kernel<T, true, 1, false> : rank_update_kernel<T, false, 1, false>);
  else if (!two)
    launch(vec ? rank_update_kernel<T, true, 2, false> : rank_update_kernel<T, false, 2, false>);
  else if (uplo == WGB_LOWER)
    launch(vec ? rank_update_kernel<T, true, 1, true> : rank_update_kernel<T, false, 1, true>);
  else
    launch(vec ? rank_update_kernel<T, true, 2, true> : rank_update_kernel<T, false, 2, true>);
  WGB_CHECK_LAUNCH("rank_update_kernel");
  wgb::timing_end(ctx);
  return WGB_OK;
}

// ssymv / dsymv: y <- alpha S x + beta y, S the n x n symmetric matrix whose
// uplo triangle A holds (column-major). The triangle is read once: block
// (r, p) takes rows [1024 r, +1024) (4 per lane in each row group, their x
// entries in registers) and panel p, columns [128 p, +128), 8 at a time with all of a
// step's loads in flight, and uses each stored element twice: A(i, j) x(j)
// for row i and, off the diagonal, A(i, j) x(i) for its mirror, row j. The
// row sums of a panel go to rowpart[p][i]; the mirror sums of a column are
// folded across each wave (shuffles) and, once at the end of the block,
// across its 4 waves (LDS) into colpart[r][j]. symv_fold_kernel then adds, for each j, exactly the slots
// the triangle's blocks wrote, in a fixed order (deterministic), and applies
// alpha and beta. Every term is taken (no zero skipping, as reference BLAS's
// symv). Blocks that cross the diagonal mask elements outside the triangle
// by selecting their terms away (never multiplying them).
// Measured at 16384 / 8192 (lower, TB/s of triangle traffic, fp32 / fp64):
// 1 row group and 128-column panels 3.5 / 3.1 and 2.1 / 2.7; 2 groups 2.8 /
// 2.9 and 1.4 / 1.8, 4 groups (4 columns a step) 2.7 / 2.3 and 0.8 / 1.0
// (fewer blocks); 64-column panels 3.3 / 3.0 and 2.5 / 2.6, 32-column 3.2 /
// 2.8 and 2.4 / 2.5.
constexpr int kSymvGroups = 1;                         // 1024-row groups per block
constexpr int kSymvRows = kSymvGroups * 4 * kThreads;  // rows per block
constexpr int kSymvPanel = 128;                        // columns per block
constexpr int kSymvStep = 8;                           // columns per step
// MODE 0: symv (row and mirror sums); 1: strmv without transpose (row sums
// over the triangle, diagonal included, a column skipped where x is zero);
// 2: strmv transposed (column sums over the triangle, diagonal included, no
// skipping). UNIT: the diagonal taken as 1, its stored value never used.
template <typename T, bool VEC, int UPLO, int MODE = 0, bool UNIT = false>
__global__ __launch_bounds__(kThreads) void symv_kernel(int64_t n, const T *__restrict__ A, int64_t lda,
                                                        const T *__restrict__ x, int64_t incx,
                                                        T *__restrict__ rowpart,
                                                        T *__restrict__ colpart) {
  typedef vec4<T> f4;
  constexpr int G = kSymvGroups, S = kSymvStep;
  const int64_t r0 = (int64_t)blockIdx.x * kSymvRows;
  const int64_t c0 = (int64_t)blockIdx.y * kSymvPanel;
  const int64_t rlast = r0 + kSymvRows - 1;
  // does the block hold any element of the triangle? (block-uniform)
  if (UPLO == 1 ? rlast < c0 : r0 > c0 + kSymvPanel - 1) return;
  const int64_t cend = c0 + kSymvPanel < n ? c0 + kSymvPanel : n;
  // a block strictly below (lower) / above (upper) the diagonal needs no
  // masks: every element stored, none on the diagonal
  const bool cross = UPLO == 1 ? r0 < cend : rlast >= c0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool whole = VEC && rlast < n;  // every lane's rows inside n
  // group g: this lane's 4 rows i0[g] .. i0[g]+3 (rows[g] of them inside n)
  int64_t i0[G], ib[G];
  int rows[G];
  f4 xv[G];
  T racc[G][4];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    i0[g] = r0 + (int64_t)g * 4 * kThreads + 4 * threadIdx.x;
    rows[g] = i0[g] >= n ? 0 : (i0[g] + 4 <= n ? 4 : (int)(n - i0[g]));
    ib[g] = rows[g] > 0 ? i0[g] : 0;  // a row inside the matrix
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      xv[g][q] = q < rows[g] ? x[(i0[g] + q) * incx] : (T)0;
      racc[g][q] = (T)0;
    }
  }
  // per-wave column sums of every step, added across the waves once at the
  // end: no barrier between steps, so a step's loads never wait on the
  // previous step's reduction
  __shared__ T red[kSymvPanel / S][4][S];
  // the step loop, compiled once per (WHOLE, CROSS): with either as a
  // run-time test the loads sat in separate branches and issued one by one
  auto steps = [&](auto whole_tag, auto cross_tag) {
    constexpr bool WHOLE = decltype(whole_tag)::value;
    constexpr bool CROSS = decltype(cross_tag)::value;
    int step = 0;
    for (int64_t j = c0; j < cend; j += S, ++step) {
      const int cols = cend - j < S ? (int)(cend - j) : S;
      f4 a[S][G];
      T xc[S];
#pragma unroll
      for (int c = 0; c < S; ++c) {
        const int64_t jc = j + (c < cols ? c : 0);  // clamped: every load in bounds
        const T xj = x[jc * incx];
        xc[c] = c < cols ? xj : (T)0;
        const T *col = A + jc * lda;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          if constexpr (WHOLE) {
            a[c][g] = ld_nt(col + i0[g]);
          } else {
            // rows past n read row ib (inside the matrix) and are never
            // used; a lane with no rows in a group (kept for the block's
            // final barrier) reads row 0
#pragma unroll
            for (int q = 0; q < 4; ++q) a[c][g][q] = col[ib[g] + (q < rows[g] ? q : 0)];
          }
        }
      }
      T cacc[S];
#pragma unroll
      for (int c = 0; c < S; ++c) {
        cacc[c] = (T)0;
        const int64_t jc = j + c;
#pragma unroll
        for (int g = 0; g < G; ++g) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int64_t i = i0[g] + q;
            bool in = c < cols && q < rows[g];  // stored element (i, jc)
            bool mirror = in;                   // ... off the diagonal
            if constexpr (CROSS) {
              in = in && (UPLO == 1 ? i >= jc : i <= jc);
              mirror = in && i != jc;
            }
            T av = a[c][g][q];
            if constexpr (UNIT && CROSS) av = i == jc ? (T)1 : av;  // only a crossing block holds the diagonal
            if constexpr (MODE == 0) {
              racc[g][q] = in ? fma(av, xc[c], racc[g][q]) : racc[g][q];
              cacc[c] = mirror ? fma(av, xv[g][q], cacc[c]) : cacc[c];
            } else if constexpr (MODE == 1) {
              // reference BLAS's column form: a zero x entry skips its column
              racc[g][q] = in && xc[c] != (T)0 ? fma(av, xc[c], racc[g][q]) : racc[g][q];
            } else {
              cacc[c] = in ? fma(av, xv[g][q], cacc[c]) : cacc[c];
            }
          }
        }
      }
      if constexpr (MODE == 1) continue;  // row sums only
      // the step's column sums across the wave
#pragma unroll
      for (int c = 0; c < S; ++c) {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) cacc[c] += __shfl_xor(cacc[c], off, 64);
      }
      if (lane < S) {
        T v = cacc[0];
#pragma unroll
        for (int c = 1; c < S; ++c) v = lane == c ? cacc[c] : v;
        red[step][wave][lane] = v;
      }
    }
  };
  if (whole && !cross)
    steps(std::true_type{}, std::false_type{});
  else if (whole)
    steps(std::true_type{}, std::true_type{});
  else
    steps(std::false_type{}, std::true_type{});
  if (MODE != 2) {
#pragma unroll
    for (int g = 0; g < G; ++g)
      for (int q = 0; q < rows[g]; ++q) rowpart[(int64_t)blockIdx.y * n + i0[g] + q] = racc[g][q];
  }
  if (MODE == 1) return;  // uniform, after the last use of red
  __syncthreads();
  if (threadIdx.x < cend - c0) {
    const int st = threadIdx.x / S, c = threadIdx.x % S;
    const T v = ((red[st][0][c] + red[st][1][c]) + red[st][2][c]) + red[st][3][c];
    colpart[(int64_t)blockIdx.x * n + c0 + threadIdx.x] = v;
  }
}

// y(j) <- alpha (sum of the row sums of the panels that reach row j + sum of
// the mirror sums of the row chunks that reach column j) + beta y(j): the
// slots symv_kernel wrote for j, lower (UPLO 1): panels 0 .. j/128, chunks
// from the one holding row 128 (j/128) on; upper: panels j/128 .. P-1, chunks
// up to the one holding row 128 (j/128) + 127. beta == 0 never reads y.
template <typename T, int UPLO, int MODE = 0>
__global__ __launch_bounds__(kThreads) void symv_fold_kernel(int64_t n, const T *__restrict__ rowpart,
                                                             const T *__restrict__ colpart, T alpha,
                                                             T beta, T *__restrict__ y, int64_t incy) {
  const int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (j >= n) return;
  const int64_t np = (n + kSymvPanel - 1) / kSymvPanel, nr = (n + kSymvRows - 1) / kSymvRows;
  const int64_t pj = j / kSymvPanel;
  const int64_t p0 = UPLO == 1 ? 0 : pj, p1 = UPLO == 1 ? pj + 1 : np;
  const int64_t ra = UPLO == 1 ? (pj * kSymvPanel) / kSymvRows : 0;
  const int64_t rb = UPLO == 1 ? nr : (pj * kSymvPanel + kSymvPanel - 1) / kSymvRows + 1;
  T s = (T)0;
  if (MODE != 2) {  // row sums (symv, strmv without transpose)
    int64_t p = p0;
    for (; p + 8 <= p1; p += 8) {
      T v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = rowpart[(p + u) * n + j];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; p < p1; ++p) s += rowpart[p * n + j];
  }
  if (MODE != 1)  // column sums (symv's mirrors, strmv transposed)
    for (int64_t r = ra; r < (rb < nr ? rb : nr); ++r) s += colpart[r * n + j];
  T v = alpha * s;
  if (beta != (T)0) v = fma(beta, y[j * incy], v);
  y[j * incy] = v;
}

template <typename T>
int symv(wgb_ctx *ctx, int uplo, int64_t n, T alpha, const T *A, int64_t lda, const T *x, int64_t incx,
         T beta, T *y, int64_t incy) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if (uplo != WGB_LOWER && uplo != WGB_UPPER)
    return fail(WGB_ERR_INVALID_VALUE, "uplo must be WGB_LOWER or WGB_UPPER");
  if (n < 0) return fail(WGB_ERR_INVALID_VALUE, "n must be non-negative");
  if (lda < imax(1, n)) return fail(WGB_ERR_INVALID_VALUE, "lda must be >= max(1, n)");
  if (incx <= 0 || incy <= 0) return fail(WGB_ERR_INVALID_VALUE, "incx and incy must be positive");
  if (n == 0) return WGB_OK;
  if (alpha == (T)0 && beta == (T)1) {
    // dsymv: reference BLAS's quick return, no kernel (src/dsymv/dsymv.mjs:116);
    // ssymv runs (and times) its kernels there (src/ssymv/ssymv.mjs): an
    // empty span, y untouched
    if (sizeof(T) == 8) return WGB_OK;
    wgb::timing_begin(ctx);
    wgb::timing_end(ctx);
    return WGB_OK;
  }
  if (!y || (alpha != (T)0 && (!A || !x))) return fail(WGB_ERR_INVALID_VALUE, "A, x or y is null");
  wgb::timing_begin(ctx);
  if (alpha == (T)0) {
    scale_y_kernel<T><<<(unsigned)cdiv(n, kThreads), kThreads, 0, ctx->stream>>>(n, beta, y, incy);
    WGB_CHECK_LAUNCH("scale_y_kernel");
    wgb::timing_end(ctx);
    return WGB_OK;
  }
  const int64_t nr = cdiv(n, kSymvRows), np = cdiv(n, kSymvPanel);
  if (np > 65535) return fail(WGB_ERR_INVALID_VALUE, "n too large for one launch");
  if ((st = wgb::ensure_op_workspace(ctx, (size_t)((np + nr) * n) * sizeof(T)))) return st;
  T *rowpart = static_cast<T *>(ctx->op_ws);
  T *colpart = rowpart + np * n;
  const dim3 grid((unsigned)nr, (unsigned)np);
  const bool vec = lda % 4 == 0 && aligned4(A);
  auto launch = [&](auto kern) {
    kern<<<grid, kThreads, 0, ctx->stream>>>(n, A, lda, x, incx, rowpart, colpart);
  };
  if (uplo == WGB_LOWER)
    launch(vec ? symv_kernel<T, true, 1> : symv_kernel<T, false, 1>);
  else
    launch(vec ? symv_kernel<T, true, 2> : symv_kernel<T, false, 2>);
  WGB_CHECK_LAUNCH("symv_kernel");
  if (uplo == WGB_LOWER)
    symv_fold_kernel<T, 1><<<(unsigned)cdiv(n, kThreads), kThreads, 0, ctx->stream>>>(
        n, rowpart, colpart, alpha, beta, y, incy);
  else
    symv_fold_kernel<T, 2><<<(unsigned)cdiv(n, kThreads), kThreads, 0, ctx->stream>>>(
        n, rowpart, colpart, alpha, beta, y, incy);
  WGB_CHECK_LAUNCH("symv_fold_kernel");
  wgb::timing_end(ctx);
  return WGB_OK;
}

// strmv / dtrmv: y <- op(T) x, T the n x n triangle (uplo) of A, unit
// diagonal taken as 1 where diag is WGB_UNIT; on symv_kernel's row sums
// (no transpose, with the column form's zero skip) or column sums
// (transpose), folded as symv's. x and y must not overlap.
template <typename T>
int trmv(wgb_ctx *ctx, int uplo, int trans, int diag, int64_t n, const T *A, int64_t lda, const T *x,
         int64_t incx, T *y, int64_t incy) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if (uplo != WGB_LOWER && uplo != WGB_UPPER)
    return fail(WGB_ERR_INVALID_VALUE, "uplo must be WGB_LOWER or WGB_UPPER");
  if (trans != WGB_NO_TRANS && trans != WGB_TRANS)
    return fail(WGB_ERR_INVALID_VALUE, "trans must be WGB_NO_TRANS or WGB_TRANS");
  if (diag != WGB_NON_UNIT && diag != WGB_UNIT)
    return fail(WGB_ERR_INVALID_VALUE, "diag must be WGB_NON_UNIT or WGB_UNIT");
  if (n < 0) return fail(WGB_ERR_INVALID_VALUE, "n must be non-negative");
  if (lda < imax(1, n)) return fail(WGB_ERR_INVALID_VALUE, "lda must be >= max(1, n)");
  if (incx <= 0 || incy <= 0) return fail(WGB_ERR_INVALID_VALUE, "incx and incy must be positive");
  if (n == 0) return WGB_OK;
  if (!A || !x || !y) return fail(WGB_ERR_INVALID_VALUE, "A, x or y is null");
  const int64_t nr = cdiv(n, kSymvRows), np = cdiv(n, kSymvPanel);
  if (np > 65535) return fail(WGB_ERR_INVALID_VALUE, "n too large for one launch");
  if ((st = wgb::ensure_op_workspace(ctx, (size_t)((np + nr) * n) * sizeof(T)))) return st;
  T *rowpart = static_cast<T *>(ctx->op_ws);
  T *colpart = rowpart + np * n;
  wgb::timing_begin(ctx);
  const dim3 grid((unsigned)nr, (unsigned)np);
  const bool vec = lda % 4 == 0 && aligned4(A);
  const bool lower = uplo == WGB_LOWER, nt = trans == WGB_NO_TRANS, unit = diag == WGB_UNIT;
  auto launch = [&](auto kern) {
    kern<<<grid, kThreads, 0, ctx->stream>>>(n, A, lda, x, incx, rowpart, colpart);
  };
  // one instantiation per (vector loads, uplo, form, unit)
  auto pick = [&](auto vec_tag, auto lower_tag, auto mode_tag, auto unit_tag) {
    launch(symv_kernel<T, decltype(vec_tag)::value, decltype(lower_tag)::value ? 1 : 2,
                       decltype(mode_tag)::value, decltype(unit_tag)::value>);
  };
  auto by_unit = [&](auto v, auto l, auto m) {
    if (unit)
      pick(v, l, m, std::true_type{});
    else
      pick(v, l, m, std::false_type{});
  };
  auto by_mode = [&](auto v, auto l) {
    if (nt)
      by_unit(v, l, std::integral_constant<int, 1>{});
    else
      by_unit(v, l, std::integral_constant<int, 2>{});
  };
  auto by_lower = [&](auto v) {
    if (lower)
      by_mode(v, std::true_type{});
    else
      by_mode(v, std::false_type{});
  };
  if (vec)
    by_lower(std::true_type{});
  else
    by_lower(std::false_type{});
  WGB_CHECK_LAUNCH("symv_kernel");
  auto fold = [&](auto kern) {
    kern<<<(unsigned)cdiv(n, kThreads), kThreads, 0, ctx->stream>>>(n, rowpart, colpart, (T)1, (T)0, y,
                                                                    incy);
  };
  if (lower)
    fold(nt ? symv_fold_kernel<T, 1, 1> : symv_fold_kernel<T, 1, 2>);
  else
    fold(nt ? symv_fold_kernel<T, 2, 1> : symv_fold_kernel<T, 2, 2>);
  WGB_CHECK_LAUNCH("symv_fold_kernel");
  wgb::timing_end(ctx);
  return WGB_OK;
}

// sgemv / dgemv on the kernels above. dgemv keeps reference BLAS's quick
// return for alpha == 0 with beta == 1 (src/dgemv/dgemv.mjs:126: no
// kernel, y untouched bit for bit); sgemv times an empty span there, as
// wgblas runs a kernel (src/sgemv/sgemv.mjs:85 returns early only for m or
// n == 0).
template <typename T>
int gemv(wgb_ctx *ctx, int trans, int64_t m, int64_t n, T alpha, const T *A, int64_t lda,
         const T *x, int64_t incx, T beta, T *y, int64_t incy) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if (trans != WGB_NO_TRANS && trans != WGB_TRANS)
    return fail(WGB_ERR_INVALID_VALUE, "trans must be WGB_NO_TRANS or WGB_TRANS");
  if (m < 0 || n < 0) return fail(WGB_ERR_INVALID_VALUE, "m and n must be non-negative");
  if (lda < imax(1, m)) return fail(WGB_ERR_INVALID_VALUE, "lda must be >= max(1, m)");
  if (incx <= 0 || incy <= 0) return fail(WGB_ERR_INVALID_VALUE, "incx and incy must be positive");
  // reference BLAS quick return: nothing to do, y untouched
  if (m == 0 || n == 0) return WGB_OK;
  if (alpha == (T)0 && beta == (T)1) {
    if (sizeof(T) == 8) return WGB_OK;
    // y untouched; this call's empty span, so per-call timing reports it
    // rather than an older call
    wgb::timing_begin(ctx);
    wgb::timing_end(ctx);
    return WGB_OK;
  }
  if (!y || (alpha != (T)0 && (!A || !x))) return fail(WGB_ERR_INVALID_VALUE, "A, x or y is null");
  const bool nt = trans == WGB_NO_TRANS;
  const int64_t len = nt ? m : n;  // length of y
  wgb::timing_begin(ctx);
  if (alpha == (T)0) {
    scale_y_kernel<T><<<(unsigned)cdiv(len, kThreads), kThreads, 0, ctx->stream>>>(len, beta, y, incy);
    WGB_CHECK_LAUNCH("scale_y_kernel");
    wgb::timing_end(ctx);
    return WGB_OK;
  }
  const bool vecA = lda % 4 == 0 && aligned4(A);
  // blocks along the output; split the contraction dimension until about
  // the target block count streams A (N: >= kMinColsN columns per split; T: >= 256
  // rows, a multiple of 256 so every split starts aligned)
  const int cpw = m <= kShortColsRows ? kColsPerWaveShort : kColsPerWave;  // T form
  const int64_t bx = nt ? cdiv(m, 4 * kThreads * kGroupsN) : cdiv(cdiv(n, cpw), kThreads / 64);
  const int64_t target = nt ? kTargetBlocksN : kTargetBlocks;
  int64_t want = bx >= target ? 1 : cdiv(target, bx);
  const int64_t most = nt ? cdiv(n, kMinColsN) : cdiv(m, 256);
  if (want > most) want = most;
  if (want > 65535) want = 65535;  // grid y limit
  if (want < 1) want = 1;
  const int64_t per = nt ? cdiv(n, want) : cdiv(cdiv(m, want), 256) * 256;
  const int64_t splits = nt ? cdiv(n, per) : cdiv(m, per);
  T *part = nullptr;
  if (splits > 1) {
    // partials, then the fold passes' group sums after them
    const int64_t groups = cdiv(splits, kFold);
    if ((st = wgb::ensure_op_workspace(ctx, (size_t)((splits + groups) * len) * sizeof(T))))
      return st;
    part = static_cast<T *>(ctx->op_ws);
  }
  dim3 grid((unsigned)bx, (unsigned)splits);
  if (nt) {
    if (vecA)
      gemv_n_kernel<T, true><<<grid, kThreads, 0, ctx->stream>>>(m, n, A, lda, x, incx, per, part,
                                                               alpha, beta, y, incy);
    else
      gemv_n_kernel<T, false><<<grid, kThreads, 0, ctx->stream>>>(m, n, A, lda, x, incx, per, part,
                                                                alpha, beta, y, incy);
    WGB_CHECK_LAUNCH("gemv_n_kernel");
  } else {
    const bool vec = vecA && incx == 1 && aligned4(x);
    auto launch = [&](auto kern) {
      kern<<<grid, kThreads, 0, ctx->stream>>>(m, n, A, lda, x, incx, per, part, alpha, beta, y, incy);
    };
    if (cpw == kColsPerWaveShort)
      launch(vec ? gemv_t_kernel<T, true, kColsPerWaveShort> : gemv_t_kernel<T, false, kColsPerWaveShort>);
    else
      launch(vec ? gemv_t_kernel<T, true, kColsPerWave> : gemv_t_kernel<T, false, kColsPerWave>);
    WGB_CHECK_LAUNCH("gemv_t_kernel");
  }
  if (part) {
    // fold passes until one group of at most kFold remains; each pass
    // alternates between the two halves of the workspace
    T *src = part, *dst = part + splits * len;
    int64_t k = splits;
    while (k > kFold) {
      const int64_t groups = cdiv(k, kFold);
      gemv_fold_kernel<T><<<dim3((unsigned)cdiv(len, kThreads), (unsigned)groups), kThreads, 0,
                         ctx->stream>>>(len, k, src, dst, alpha, beta, y, incy);
      WGB_CHECK_LAUNCH("gemv_fold_kernel");
      T *t = src;
      src = dst;
      dst = t;
      k = groups;
    }
    gemv_fold_kernel<T><<<dim3((unsigned)cdiv(len, kThreads), 1), kThreads, 0, ctx->stream>>>(
        len, k, src, nullptr, alpha, beta, y, incy);
    WGB_CHECK_LAUNCH("gemv_fold_kernel");
  }
  wgb::timing_end(ctx);
  return WGB_OK;
}

}  // namespace

extern "C" int wgb_sgemv(wgb_ctx *ctx, int trans, int64_t m, int64_t n, float alpha,
                         const float *A, int64_t lda, const float *x, int64_t incx, float beta,
                         float *y, int64_t incy) {
  return gemv<float>(ctx, trans, m, n, alpha, A, lda, x, incx, beta, y, incy);
}

extern "C" int wgb_sger(wgb_ctx *ctx, int64_t m, int64_t n, float alpha, const float *x,
                        int64_t incx, const float *y, int64_t incy, float *A, int64_t lda) {
  return rank_update<float>(ctx, 0, false, m, n, alpha, x, incx, y, incy, A, lda);
}

extern "C" int wgb_dger(wgb_ctx *ctx, int64_t m, int64_t n, double alpha, const double *x,
                        int64_t incx, const double *y, int64_t incy, double *A, int64_t lda) {
  return rank_update<double>(ctx, 0, false, m, n, alpha, x, incx, y, incy, A, lda);
}

extern "C" int wgb_ssyr(wgb_ctx *ctx, int uplo, int64_t n, float alpha, const float *x,
                        int64_t incx, float *A, int64_t lda) {
  if (uplo == 0) return fail(WGB_ERR_INVALID_VALUE, "uplo must be WGB_LOWER or WGB_UPPER");
  return rank_update<float>(ctx, uplo, false, n, n, alpha, x, incx, x, incx, A, lda);
}

extern "C" int wgb_dsyr(wgb_ctx *ctx, int uplo, int64_t n, double alpha, const double *x,
                        int64_t incx, double *A, int64_t lda) {
  if (uplo == 0) return fail(WGB_ERR_INVALID_VALUE, "uplo must be WGB_LOWER or WGB_UPPER");
  return rank_update<double>(ctx, uplo, false, n, n, alpha, x, incx, x, incx, A, lda);
}

extern "C" int wgb_ssyr2(wgb_ctx *ctx, int uplo, int64_t n, float alpha, const float *x,
                         int64_t incx, const float *y, int64_t incy, float *A, int64_t lda) {
  if (uplo == 0) return fail(WGB_ERR_INVALID_VALUE, "uplo must be WGB_LOWER or WGB_UPPER");
  return rank_update<float>(ctx, uplo, true, n, n, alpha, x, incx, y, incy, A, lda);
}

extern "C" int wgb_dsyr2(wgb_ctx *ctx, int uplo, int64_t n, double alpha, const double *x,
                         int64_t incx, const double *y, int64_t incy, double *A, int64_t lda) {
  if (uplo == 0) return fail(WGB_ERR_INVALID_VALUE, "uplo must be WGB_LOWER or WGB_UPPER");
  return rank_update<double>(ctx, uplo, true, n, n, alpha, x, incx, y, incy, A, lda);
}

extern "C" int wgb_ssymv(wgb_ctx *ctx, int uplo, int64_t n, float alpha, const float *A,
                         int64_t lda, const float *x, int64_t incx, float beta, float *y,
                         int64_t incy) {
  return symv<float>(ctx, uplo, n, alpha, A, lda, x, incx, beta, y, incy);
}

extern "C" int wgb_dsymv(wgb_ctx *ctx, int uplo, int64_t n, double alpha, const double *A,
                         int64_t lda, const double *x, int64_t incx, double beta, double *y,
                         int64_t incy) {
  return symv<double>(ctx, uplo, n, alpha, A, lda, x, incx, beta, y, incy);
}

extern "C" int wgb_strmv(wgb_ctx *ctx, int uplo, int trans, int diag, int64_t n, const float *A,
                         int64_t lda, const float *x, int64_t incx, float *y, int64_t incy) {
  return trmv<float>(ctx, uplo, trans, diag, n, A, lda, x, incx, y, incy);
}

extern "C" int wgb_dtrmv(wgb_ctx *ctx, int uplo, int trans, int diag, int64_t n, const double *A,
                         int64_t lda, const double *x, int64_t incx, double *y, int64_t incy) {
  return trmv<double>(ctx, uplo, trans, diag, n, A, lda, x, incx, y, incy);
}

extern "C" int wgb_dgemv(wgb_ctx *ctx, int trans, int64_t m, int64_t n, double alpha,
                         const double *A, int64_t lda, const double *x, int64_t incx, double beta,
                         double *y, int64_t incy) {
  return gemv<double>(ctx, trans, m, n, alpha, A, lda, x, incx, beta, y, incy);
}
