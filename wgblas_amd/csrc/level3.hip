// The level-3 routines that run on the GEMM kernel: ssyr2k, ssymm, strmm,
// strsm (wgblas src/{ssyr2k,ssymm,strmm,strsm}/*.mjs).
//
// ssyr2k: two triangle GEMM launches, the second with beta = 1.
// ssymm: the symmetric operand is expanded into a dense workspace copy
//   (LDS-tiled, coalesced both ways), then one GEMM.
// strmm: A's triangle is copied with zeros elsewhere, B is copied (the GEMM
//   cannot read and write B at once), then one GEMM whose tiles only run the
//   k-tiles the triangle reaches (about half the flops of a dense product).
// strsm: recursive halving of the triangular dimension. Diagonal blocks of
//   order <= 128 are solved by substitution, one lane per right-hand side,
//   eight waves splitting its unknowns; the off-diagonal updates are GEMMs that
//   read the solved rows of B and write other rows of B in place (disjoint
//   memory), so strsm needs no workspace and no explicit inverse.
#include "common.h"

#include <hip/hip_runtime.h>

#include "wgblas_hip.h"

namespace {

using wgb::fail;

constexpr int kTile = 64;  // symmetrize tile (64 x 64)
constexpr int kLeaf = 128;  // order of strsm's substitution blocks

int64_t imax(int64_t a, int64_t b) { return a > b ? a : b; }
int64_t round4(int64_t v) { return (v + 3) / 4 * 4; }

// W (order x order, column-major, ld ldw) <- the symmetric matrix whose uplo
// triangle A holds (src/shaders/symmetrize.wgsl). Block (bi, bj) writes W's
// 64 x 64 tile (bi, bj): a tile inside the stored triangle copies A's tile,
// a tile in the other triangle reads the mirrored tile (bj, bi) and
// transposes it through LDS, a diagonal tile takes each element from
// whichever of (i, j), (j, i) is stored. 256 threads = 64 rows x 4 column
// phases, so every wave reads and writes 256 contiguous bytes of a column.
__global__ __launch_bounds__(256) void symmetrize_kernel(int64_t order, const float *__restrict__ A,
                                                         int64_t lda, int uplo,
                                                         float *__restrict__ W, int64_t ldw) {
  __shared__ float s[kTile][kTile + 1];  // s[col][row] of the source tile
  const int bi = blockIdx.x, bj = blockIdx.y;
  const bool lower = uplo == WGB_LOWER;
  const bool diag = bi == bj;
  const bool stored = lower ? bi > bj : bi < bj;
  const int si = (stored || diag) ? bi : bj, sj = (stored || diag) ? bj : bi;
  const int r = threadIdx.x & 63, ph = threadIdx.x >> 6;
  const int64_t srow = (int64_t)si * kTile + r;
  // unconditional loads from clamped addresses, all in flight together
  float v[kTile / 4];
#pragma unroll
  for (int q = 0; q < kTile / 4; ++q) {
    const int64_t scol = (int64_t)sj * kTile + ph + 4 * q;
    const bool ok = srow < order && scol < order;
    v[q] = A[(ok ? srow : 0) + (ok ? scol : 0) * lda];
  }
#pragma unroll
  for (int q = 0; q < kTile / 4; ++q) {
    const int64_t scol = (int64_t)sj * kTile + ph + 4 * q;
    s[ph + 4 * q][r] = (srow < order && scol < order) ? v[q] : 0.f;
  }
  __syncthreads();
  const int64_t row = (int64_t)bi * kTile + r;
  if (row >= order) return;
  for (int c = ph; c < kTile; c += 4) {
    const int64_t col = (int64_t)bj * kTile + c;
    if (col >= order) break;
    float v;
    if (stored)
      v = s[c][r];
    else if (!diag)
      v = s[r][c];  // W(row, col) = A(col, row), element (c, r) of tile (bj, bi)
    else
      v = (lower ? r >= c : r <= c) ? s[c][r] : s[r][c];
    W[row + col * ldw] = v;
  }
}

// W <- A's uplo triangle, zero elsewhere, ones on the diagonal for a unit
// triangle (src/shaders/triangularize.wgsl builds op(A); W keeps A's own
// orientation and the GEMM applies transA).
// A thread writes 4 consecutive rows of W (one 16-byte store; W's ld is a
// multiple of 4) in columns blockIdx.y, blockIdx.y + gridDim.y, ...; a row
// group wholly outside the triangle writes zeros without reading A. VEC: lda
// a multiple of 4 and A 16-byte aligned (16-byte loads).
template <bool VEC>
__global__ __launch_bounds__(256) void triangle_copy_kernel(int64_t order,
                                                            const float *__restrict__ A,
                                                            int64_t lda, int uplo, int unit,
                                                            float *__restrict__ W, int64_t ldw) {
  typedef float F4 __attribute__((ext_vector_type(4)));
  const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (row >= order) return;
  const bool lower = uplo == WGB_LOWER;
  const int nr = order - row < 4 ? (int)(order - row) : 4;
  for (int64_t col = blockIdx.y; col < order; col += gridDim.y) {
    // does any of rows row .. row+nr-1 lie in the triangle (diagonal included)?
    const bool any = lower ? row + nr - 1 >= col : row <= col;
    F4 v = F4(0.f);
    if (any) {
      const float *a = A + row + col * lda;
      if (VEC && nr == 4) {
        v = *reinterpret_cast<const F4 *>(a);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = a[c < nr ? c : 0];
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int64_t r = row + c;
        if (r == col)
          v[c] = unit ? 1.f : v[c];
        else if (!(lower ? r > col : r < col))
          v[c] = 0.f;  // the other triangle: never used, whatever it holds
      }
    }
    float *w = W + row + col * ldw;
    if (nr == 4) {
      *reinterpret_cast<F4 *>(w) = v;
    } else {
      for (int c = 0; c < nr; ++c) w[c] = v[c];
    }
  }
}

// Substitution solve of one diagonal block, in the solve frame: for every
// right-hand side v, M x = alpha v with M lower triangular of order nb <= NB.
// Frame element (i, k) of M is Ablk[ia(i) mi + ia(k) mk] and element i of
// right-hand side r is Bblk[ia(i) vi + r vr], where ia(i) = nb-1-i for an
// upper system solved backward (rev) and i otherwise; the solution
// overwrites v.
//
// A block takes 64 right-hand sides, one per lane, and its NB / 16 waves
// each own 16 consecutive rows of them in registers. Chunk c: wave c
// substitutes through its rows (x_k *= 1/M(k,k), then x_i -= M(i,k) x_k for
// its later rows: the column-oriented order of wgblas's strsm_small.wgsl and
// of reference BLAS) and publishes them to LDS; after one barrier every later
// wave subtracts the chunk's contribution from its rows. M's entries are LDS
// broadcasts and the block needs one barrier per chunk. The diagonal's
// reciprocals are formed once per block: x * RN(1/d) is within two ulps of
// x / d, and zero, infinite and NaN diagonals give the quotient's special
// values (only a diagonal below 2^-126 in magnitude, whose reciprocal
// overflows, differs). alpha is applied as v is read. Rows past nb are
// padding with a unit diagonal and zero right-hand side; they never feed real
// rows. Loads are unconditional, from addresses clamped into the block, so
// that all of them are in flight together (a guarded load is waited for
// before the next one issues).
template <int NB>
__global__ __launch_bounds__(4 * NB) void trsm_leaf_kernel(int nb, int64_t nrhs,
                                                          const float *__restrict__ Ablk, int64_t mi,
                                                          int64_t mk, int rev, int unit,
                                                          float *__restrict__ Bblk, int64_t vi,
                                                          int64_t vr, float alpha) {
  constexpr int kThreadsLeaf = 4 * NB;       // NB / 16 waves
  constexpr int kSplit = NB / 16;            // waves = row chunks
  constexpr int kRows = 16;                  // rows per wave
  constexpr int kPer = NB * NB / kThreadsLeaf;
  constexpr int kGroups = kThreadsLeaf / NB;  // left-side staging: column groups (4)
  constexpr int kCols = 64 / kGroups;         // right-hand sides per column group (16)
  static_assert(kCols == kRows, "one staging register set serves both sides");
  __shared__ __attribute__((aligned(16))) float Ms[NB * NB];  // Ms[k*NB + i] = M(i, k)
  __shared__ float Xs[NB][65];                                // Xs[i][rhs]
  __shared__ float Rd[NB];                                    // 1 / M(k, k)
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int row0 = wave * kRows;
  const int64_t rhs0 = (int64_t)blockIdx.x * 64;
  const int64_t r = rhs0 + lane;  // this lane's right-hand side
  const bool left = vi == 1;      // the frame index is B's contiguous one
  const int si = t % NB, sg = t / NB;  // left-side staging: frame index, column group

  // ---- every global load first
  float mv[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int e = t + q * kThreadsLeaf;
    const int i = e % NB, k = e / NB;
    const bool in = i < nb && k <= i;
    const int ii = in ? (rev ? nb - 1 - i : i) : 0, kk = in ? (rev ? nb - 1 - k : k) : 0;
    mv[q] = Ablk[ii * mi + kk * mk];
  }
  // left: thread (si, sg) loads frame index si of right-hand sides sg,
  // sg + kGroups, ...; right: lane = right-hand side, wave w its 16 rows
  float bv[kRows];
#pragma unroll
  for (int q = 0; q < kRows; ++q) {
    int64_t at;
    if (left) {
      const int64_t rc = rhs0 + sg + q * kGroups;
      at = (si < nb ? (rev ? nb - 1 - si : si) : 0) + (rc < nrhs ? rc : 0) * vr;
    } else {
      const int i = row0 + q;
      at = (int64_t)(i < nb ? (rev ? nb - 1 - i : i) : 0) * vi + (r < nrhs ? r : 0);
    }
    bv[q] = Bblk[at];
  }

  // ---- M (zero above the diagonal, unit diagonal for padding rows) and
  // the reciprocals of its diagonal into LDS
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int e = t + q * kThreadsLeaf;
    const int i = e % NB, k = e / NB;
    const bool in = i < nb && k <= i;
    const float v = i == k ? ((unit || !in) ? 1.f : mv[q]) : (in ? mv[q] : 0.f);
    Ms[e] = v;
    if (i == k) Rd[k] = 1.f / v;
  }
  float x[kRows];
  if (left) {
#pragma unroll
    for (int q = 0; q < kRows; ++q) {
      const int c = sg + q * kGroups;
      Xs[si][c] = (si < nb && rhs0 + c < nrhs) ? bv[q] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kRows; ++j) x[j] = alpha * Xs[row0 + j][lane];
  } else {
#pragma unroll
    for (int j = 0; j < kRows; ++j) x[j] = (r < nrhs && row0 + j < nb) ? alpha * bv[j] : 0.f;
  }
  __syncthreads();  // Ms and Rd complete; every read of the staged block done

  // ---- chunked substitution
  for (int c = 0; c < kSplit; ++c) {  // block-uniform chunk loop
    if (wave == c) {
#pragma unroll
      for (int j = 0; j < kRows; ++j) {
        const int k = row0 + j;
        x[j] = x[j] * Rd[k];
#pragma unroll
        for (int jj = j + 1; jj < kRows; ++jj) x[jj] = fmaf(-Ms[k * NB + row0 + jj], x[j], x[jj]);
        Xs[k][lane] = x[j];
      }
    }
    __syncthreads();
    if (wave > c) {
#pragma unroll 4
      for (int kk = 0; kk < kRows; ++kk) {
        const int k = c * kRows + kk;
        const float xk = Xs[k][lane];
#pragma unroll
        for (int j = 0; j < kRows; ++j) x[j] = fmaf(-Ms[k * NB + row0 + j], xk, x[j]);
      }
    }
  }

  // ---- write back (Xs holds every solved row: the last chunk was
  // published before the loop's final barrier)
  if (left) {
    const bool ok = si < nb;
    const int64_t at = rev ? nb - 1 - si : si;
#pragma unroll
    for (int q = 0; q < kRows; ++q) {
      const int c = sg + q * kGroups;
      const int64_t rc = rhs0 + c;
      if (ok && rc < nrhs) Bblk[at + rc * vr] = Xs[si][c];
    }
  } else if (r < nrhs) {
#pragma unroll
    for (int j = 0; j < kRows; ++j) {
      const int i = row0 + j;
      if (i < nb) Bblk[(int64_t)(rev ? nb - 1 - i : i) * vi + r] = x[j];
    }
  }
}

// strsm in the solve frame: frame index = B's row (left side) or column
// (right side); M = op(A) (left) or op(A)^T (right), lower when the solve
// runs forward.
struct Trsm {
  wgb_ctx *ctx;
  bool left, trans, unit, forward;
  int64_t m, n;
  float alpha;
  const float *A;
  int64_t lda;
  float *B;
  int64_t ldb;
};

int trsm_leaf(const Trsm &p, int64_t lo, int64_t nb, float alpha) {
  const bool m_is_a = p.left != p.trans;  // M is A itself, else A^T
  const float *Ablk = p.A + lo + lo * p.lda;
  const int64_t mi = m_is_a ? 1 : p.lda, mk = m_is_a ? p.lda : 1;
  const int64_t nrhs = p.left ? p.n : p.m;
  const int64_t grid = (nrhs + 63) / 64;
  const int rev = p.forward ? 0 : 1;
  // left: frame index = row of B (stride 1), right-hand side = column;
  // right: frame index = column of B, right-hand side = row
  float *Bblk = p.left ? p.B + lo : p.B + lo * p.ldb;
  const int64_t vi = p.left ? 1 : p.ldb, vr = p.left ? p.ldb : 1;
  trsm_leaf_kernel<kLeaf><<<(unsigned)grid, 4 * kLeaf, 0, p.ctx->stream>>>(
      (int)nb, nrhs, Ablk, mi, mk, rev, p.unit, Bblk, vi, vr, alpha);
  WGB_CHECK_LAUNCH("trsm_leaf_kernel");
  return WGB_OK;
}

// Frame rows [b, b+nbr) <- beta * themselves - M[b.., a..] X[a.., :], X the
// solved frame rows [a, a+nar). Left: B[b,:] = beta B[b,:] - op(A)[b,a] B[a,:];
// right: B[:,b] = beta B[:,b] - B[:,a] op(A)[a,b]. Both read rows / columns
// of B disjoint from the ones they write.
int trsm_update(const Trsm &p, int64_t a, int64_t nar, int64_t b, int64_t nbr, float beta) {
  const int t = p.trans ? WGB_TRANS : WGB_NO_TRANS;
  if (p.left) {
    const float *Ap = p.trans ? p.A + a + b * p.lda : p.A + b + a * p.lda;
    return wgb::gemm_f32(p.ctx, 0, t, WGB_NO_TRANS, nbr, p.n, nar, -1.f, Ap, p.lda, p.B + a, p.ldb,
                         beta, p.B + b, p.ldb, wgb::kBandNone);
  }
  const float *Ap = p.trans ? p.A + b + a * p.lda : p.A + a + b * p.lda;
  return wgb::gemm_f32(p.ctx, 0, WGB_NO_TRANS, t, p.m, nbr, nar, -1.f, p.B + a * p.ldb, p.ldb, Ap,
                       p.lda, beta, p.B + b * p.ldb, p.ldb, wgb::kBandNone);
}

// Solves frame rows [lo, hi); `scaled`: those rows of B already carry alpha.
// The first half in solve order is solved, the second half is updated with
// it (beta = alpha folds the scaling into that GEMM), then solved.
int trsm_solve(const Trsm &p, int64_t lo, int64_t hi, bool scaled) {
  const int64_t size = hi - lo;
  if (size <= kLeaf) return trsm_leaf(p, lo, size, scaled ? 1.f : p.alpha);
  const int64_t mid = lo + (size / 2 + kLeaf - 1) / kLeaf * kLeaf;
  const int64_t a0 = p.forward ? lo : mid, a1 = p.forward ? mid : hi;
  const int64_t b0 = p.forward ? mid : lo, b1 = p.forward ? hi : mid;
  int st = trsm_solve(p, a0, a1, scaled);
  if (st) return st;
  if ((st = trsm_update(p, a0, a1 - a0, b0, b1 - b0, scaled ? 1.f : p.alpha))) return st;
  return trsm_solve(p, b0, b1, true);
}

// B <- 0 over its m x n part, reading nothing.
int zero_b(wgb_ctx *ctx, int64_t m, int64_t n, float *B, int64_t ldb) {
  return wgb::gemm_f32(ctx, 0, WGB_NO_TRANS, WGB_NO_TRANS, m, n, 0, 0.f, nullptr, 1, nullptr, 1,
                       0.f, B, ldb, wgb::kBandNone);
}

int check_tri(int side, int uplo, int transA, int diag, int64_t m, int64_t n, const void *A,
              int64_t lda, const void *B, int64_t ldb) {
  if (side != WGB_LEFT && side != WGB_RIGHT)
    return fail(WGB_ERR_INVALID_VALUE, "side must be WGB_LEFT or WGB_RIGHT");
  if (uplo != WGB_LOWER && uplo != WGB_UPPER)
    return fail(WGB_ERR_INVALID_VALUE, "uplo must be WGB_LOWER or WGB_UPPER");
  if (transA != WGB_NO_TRANS && transA != WGB_TRANS)
    return fail(WGB_ERR_INVALID_VALUE, "transA must be WGB_NO_TRANS or WGB_TRANS");
  if (diag != WGB_NON_UNIT && diag != WGB_UNIT)
    return fail(WGB_ERR_INVALID_VALUE, "diag must be WGB_NON_UNIT or WGB_UNIT");
  if (m < 0 || n < 0) return fail(WGB_ERR_INVALID_VALUE, "m and n must be non-negative");
  if (m > INT32_MAX || n > INT32_MAX) return fail(WGB_ERR_INVALID_VALUE, "m and n must be below 2^31");
  const int64_t order = side == WGB_LEFT ? m : n;
  if (lda < imax(1, order)) return fail(WGB_ERR_INVALID_VALUE, "lda must be >= max(1, order of A)");
  if (ldb < imax(1, m)) return fail(WGB_ERR_INVALID_VALUE, "ldb must be >= max(1, m)");
  if (m > 0 && n > 0 && (!A || !B)) return fail(WGB_ERR_INVALID_VALUE, "A or B is null");
  return WGB_OK;
}

}  // namespace

extern "C" int wgb_ssyr2k(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t n, int64_t k,
                          float alpha, const float *A, int64_t lda, const float *B, int64_t ldb,
                          float beta, float *C, int64_t ldc) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if (transA != WGB_NO_TRANS && transA != WGB_TRANS)
    return fail(WGB_ERR_INVALID_VALUE, "transA must be WGB_NO_TRANS or WGB_TRANS");
  if (transB != WGB_NO_TRANS && transB != WGB_TRANS)
    return fail(WGB_ERR_INVALID_VALUE, "transB must be WGB_NO_TRANS or WGB_TRANS");
  // op(X)^T as the second GEMM operand: the opposite flag
  const int tAt = transA == WGB_NO_TRANS ? WGB_TRANS : WGB_NO_TRANS;
  const int tBt = transB == WGB_NO_TRANS ? WGB_TRANS : WGB_NO_TRANS;
  if ((st = wgb::check_gemm(uplo, true, transA, tBt, n, n, k, A, lda, B, ldb, C, ldc))) return st;
  if (n == 0) return WGB_OK;
  wgb::timing_begin(ctx);
  // pass 1: alpha op(A) op(B)^T + beta C; pass 2: alpha op(B) op(A)^T + C
  // (src/ssyr2k/ssyr2k.mjs:206-262), one timed span
  if ((st = wgb::gemm_f32(ctx, uplo, transA, tBt, n, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                          wgb::kBandNone)))
    return st;
  if (alpha != 0.f && k != 0 &&
      (st = wgb::gemm_f32(ctx, uplo, transB, tAt, n, n, k, alpha, B, ldb, A, lda, 1.f, C, ldc,
                          wgb::kBandNone)))
    return st;
  wgb::timing_end(ctx);
  return WGB_OK;
}

extern "C" int wgb_ssymm(wgb_ctx *ctx, int side, int uplo, int transB, int64_t m, int64_t n,
                         float alpha, const float *A, int64_t lda, const float *B, int64_t ldb,
                         float beta, float *C, int64_t ldc) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if (side != WGB_LEFT && side != WGB_RIGHT)
    return fail(WGB_ERR_INVALID_VALUE, "side must be WGB_LEFT or WGB_RIGHT");
  if (uplo != WGB_LOWER && uplo != WGB_UPPER)
    return fail(WGB_ERR_INVALID_VALUE, "uplo must be WGB_LOWER or WGB_UPPER");
  if (transB != WGB_NO_TRANS && transB != WGB_TRANS)
    return fail(WGB_ERR_INVALID_VALUE, "transB must be WGB_NO_TRANS or WGB_TRANS");
  if (m < 0 || n < 0) return fail(WGB_ERR_INVALID_VALUE, "m and n must be non-negative");
  if (m > INT32_MAX || n > INT32_MAX) return fail(WGB_ERR_INVALID_VALUE, "m and n must be below 2^31");
  const int64_t order = side == WGB_LEFT ? m : n;
  if (lda < imax(1, order)) return fail(WGB_ERR_INVALID_VALUE, "lda must be >= max(1, order of A)");
  // op(B) is m x n: B is stored m x n, or n x m when transB
  if (ldb < imax(1, transB == WGB_NO_TRANS ? m : n))
    return fail(WGB_ERR_INVALID_VALUE, "ldb must be >= max(1, rows of B)");
  if (ldc < imax(1, m)) return fail(WGB_ERR_INVALID_VALUE, "ldc must be >= max(1, m)");
  if (m == 0 || n == 0) return WGB_OK;
  if (!C || (alpha != 0.f && (!A || !B))) return fail(WGB_ERR_INVALID_VALUE, "A, B or C is null");
  wgb::timing_begin(ctx);
  if (alpha == 0.f) {
    // C <- beta C, reading neither A nor B
    st = wgb::gemm_f32(ctx, 0, WGB_NO_TRANS, WGB_NO_TRANS, m, n, 0, 0.f, nullptr, 1, nullptr, 1,
                       beta, C, ldc, wgb::kBandNone);
  } else {
    const int64_t ldw = round4(order);
    if ((st = wgb::ensure_op_workspace(ctx, (size_t)ldw * order * sizeof(float)))) return st;
    float *W = static_cast<float *>(ctx->op_ws);
    const int64_t tiles = (order + kTile - 1) / kTile;
    symmetrize_kernel<<<dim3((unsigned)tiles, (unsigned)tiles), 256, 0, ctx->stream>>>(order, A, lda,
                                                                                      uplo, W, ldw);
    WGB_CHECK_LAUNCH("symmetrize_kernel");
    st = side == WGB_LEFT
             ? wgb::gemm_f32(ctx, 0, WGB_NO_TRANS, transB, m, n, m, alpha, W, ldw, B, ldb, beta, C,
                             ldc, wgb::kBandNone)
             : wgb::gemm_f32(ctx, 0, transB, WGB_NO_TRANS, m, n, n, alpha, B, ldb, W, ldw, beta, C,
                             ldc, wgb::kBandNone);
  }
  if (st) return st;
  wgb::timing_end(ctx);
  return WGB_OK;
}

extern "C" int wgb_strmm(wgb_ctx *ctx, int side, int uplo, int transA, int diag, int64_t m,
                         int64_t n, float alpha, const float *A, int64_t lda, float *B,
                         int64_t ldb) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_tri(side, uplo, transA, diag, m, n, A, lda, B, ldb))) return st;
  if (m == 0 || n == 0) return WGB_OK;
  wgb::timing_begin(ctx);
  if (alpha == 0.f) {
    st = zero_b(ctx, m, n, B, ldb);
  } else {
    const bool left = side == WGB_LEFT;
    const int64_t order = left ? m : n;
    const int64_t ldw = round4(order), ldbc = round4(m);
    if ((st = wgb::ensure_op_workspace(ctx, (size_t)(ldw * order + ldbc * n) * sizeof(float)))) return st;
    float *W = static_cast<float *>(ctx->op_ws);
    float *Bc = W + ldw * order;  // 16-byte aligned: ldw is a multiple of 4
    const int64_t gy = order < 4096 ? order : 4096;
    const dim3 grid((unsigned)((order + 1023) / 1024), (unsigned)gy);
    if (lda % 4 == 0 && wgb::aligned16(A))
      triangle_copy_kernel<true><<<grid, 256, 0, ctx->stream>>>(order, A, lda, uplo, diag == WGB_UNIT, W, ldw);
    else
      triangle_copy_kernel<false><<<grid, 256, 0, ctx->stream>>>(order, A, lda, uplo, diag == WGB_UNIT, W, ldw);
    WGB_CHECK_LAUNCH("triangle_copy_kernel");
    WGB_CHECK_HIP(hipMemcpy2DAsync(Bc, (size_t)ldbc * sizeof(float), B, (size_t)ldb * sizeof(float),
                                   (size_t)m * sizeof(float), (size_t)n, hipMemcpyDeviceToDevice,
                                   ctx->stream));
    const bool op_lower = (uplo == WGB_LOWER) != (transA == WGB_TRANS);
    st = left ? wgb::gemm_f32(ctx, 0, transA, WGB_NO_TRANS, m, n, m, alpha, W, ldw, Bc, ldbc, 0.f, B,
                              ldb, op_lower ? wgb::kBandALower : wgb::kBandAUpper)
              : wgb::gemm_f32(ctx, 0, WGB_NO_TRANS, transA, m, n, n, alpha, Bc, ldbc, W, ldw, 0.f, B,
                              ldb, op_lower ? wgb::kBandBLower : wgb::kBandBUpper);
  }
  if (st) return st;
  wgb::timing_end(ctx);
  return WGB_OK;
}

extern "C" int wgb_strsm(wgb_ctx *ctx, int side, int uplo, int transA, int diag, int64_t m,
                         int64_t n, float alpha, const float *A, int64_t lda, float *B,
                         int64_t ldb) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_tri(side, uplo, transA, diag, m, n, A, lda, B, ldb))) return st;
  if (m == 0 || n == 0) return WGB_OK;
  wgb::timing_begin(ctx);
  if (alpha == 0.f) {
    // B becomes a literal zero, not 0 * B (src/strsm/strsm.mjs:424-430)
    st = zero_b(ctx, m, n, B, ldb);
  } else {
    Trsm p;
    p.ctx = ctx;
    p.left = side == WGB_LEFT;
    p.trans = transA == WGB_TRANS;
    p.unit = diag == WGB_UNIT;
    const bool op_lower = (uplo == WGB_LOWER) != p.trans;
    p.forward = p.left ? op_lower : !op_lower;
    p.m = m;
    p.n = n;
    p.alpha = alpha;
    p.A = A;
    p.lda = lda;
    p.B = B;
    p.ldb = ldb;
    st = trsm_solve(p, 0, p.left ? m : n, false);
  }
  if (st) return st;
  wgb::timing_end(ctx);
  return WGB_OK;
}
