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
//   order <= 256 are solved by substitution, 16 lanes per right-hand side
//   exchanging solved unknowns by DPP broadcasts; the off-diagonal updates are GEMMs that
//   read the solved rows of B and write other rows of B in place (disjoint
//   memory). The diagonal blocks are packed once per call into the operand
//   workspace; no explicit inverse is formed.
#include "common.h"

#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>

#include "wgblas_hip.h"

namespace {

using wgb::fail;

constexpr int kTile = 64;  // symmetrize tile (64 x 64)
constexpr int kLeaf = 256;  // order of strsm's substitution blocks
typedef float Vec4 __attribute__((ext_vector_type(4)));  // a native 16-byte vector

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

// Compile-time loop: f(std::integral_constant<int, I>{}) for I = 0 .. N-1.
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Lane L of every 16-lane row of the wave, copied to the row's 16 lanes
// (DPP row_newbcast).
template <int L>
__device__ __forceinline__ float row_bcast(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x150 + L, 0xf, 0xf, false));
}

// strsm's diagonal blocks in the layout trsm_leaf_kernel stages in LDS: the
// solve frame splits into blocks of kLeaf rows (the last one nb < kLeaf
// rows), and block l's image is kImg floats at P + l kImg: P[k kLeaf + i] =
// M(i, k) for k < i < nb (zero elsewhere, the diagonal included), then
// P[kLeaf^2 + k] = 1 / M(k, k) (1 for a unit diagonal and for padding rows).
// Frame element (i, k) of block l's M is Ablk[ia(i) mi + ia(k) mk], Ablk at
// A + kLeaf l (1 + lda), where ia(i) = nb-1-i for an upper system solved
// backward (rev) and i otherwise. Block (l, c) packs columns 16c .. 16c+15 of
// image l through an LDS tile: read with the stride-1 index fastest, written
// with i fastest. The diagonal's reciprocals are formed once here: x * RN(1/d)
// is within two ulps of x / d, and zero, infinite and NaN diagonals give the
// quotient's special values (only a diagonal below 2^-126 in magnitude, whose
// reciprocal overflows, differs).
constexpr int kImg = kLeaf * kLeaf + kLeaf;

__global__ __launch_bounds__(256) void trsm_pack_kernel(int64_t order, const float *__restrict__ A,
                                                        int64_t lda, int64_t mi, int64_t mk, int rev,
                                                        int unit, float *__restrict__ P) {
  __shared__ float T[16][kLeaf + 1];
  const int t = threadIdx.x, c = blockIdx.y;
  const int64_t l = blockIdx.x, lo = l * kLeaf;
  const int nb = (int)(order - lo < kLeaf ? order - lo : kLeaf);
  const float *Ablk = A + lo + lo * lda;
  const bool kfast = mk == 1;  // consecutive k are adjacent in memory
  constexpr int kQ = 16 * kLeaf / 256;  // elements per thread
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
    const int e = t + 256 * q;
    const int i = kfast ? e / 16 : e % kLeaf, kl = kfast ? e % 16 : e / kLeaf;
    const int k = 16 * c + kl;
    const bool in = i < nb && k <= i;
    const int64_t ii = in ? (rev ? nb - 1 - i : i) : 0, kk = in ? (rev ? nb - 1 - k : k) : 0;
    const float v = Ablk[ii * mi + kk * mk];
    T[kl][i] = in ? v : 0.f;
  }
  __syncthreads();
  float *img = P + l * kImg;
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
    const int e = t + 256 * q;
    const int i = e % kLeaf, kl = e / kLeaf, k = 16 * c + kl;
    img[k * kLeaf + i] = i > k ? T[kl][i] : 0.f;
  }
  if (t < 16) {
    const int k = 16 * c + t;
    img[kLeaf * kLeaf + k] = 1.f / ((unit || k >= nb) ? 1.f : T[t][k]);
  }
}

// Substitution solve of one diagonal block, in the solve frame: for every
// right-hand side v, M x = alpha v with M lower triangular of order
// nb <= kLeaf, given as its image `img` (trsm_pack_kernel). Element i of
// right-hand side r is Bblk[ia(i) vi + r vr], where ia(i) = nb-1-i for an
// upper system solved backward (rev) and i otherwise; the solution
// overwrites v.
//
// Each 16-lane row of a wave owns R right-hand sides; lane j of the row
// holds frame rows j, j+16, ..., j+240 of them in registers (x[h][g] is row
// 16g + j of right-hand side h). Step k, in the column-oriented order of
// wgblas's strsm_small.wgsl and of reference BLAS: x_k = x_k * (1 / M(k,k)),
// computed by every lane on its register of row k's group and broadcast from
// lane k % 16 across the row; then every lane subtracts M(i,k) x_k from each
// of its rows i (one fused multiply-add each). The rows i <= k that step k
// also touches are already solved (each lane keeps its row of the group as
// it is broadcast and stores it when the group ends) and M(i,k) is zero
// there, so what the update leaves in them is never read. Per row the operations are those of substitution: the
// products are subtracted in k order, then the row is scaled by the
// diagonal's reciprocal. alpha is applied as v is read. Rows past nb are
// padding with a unit diagonal and zero right-hand side; they never feed
// real rows.
//
// Scheduling. A wave solves its right-hand sides alone: x_k moves between
// lanes by one DPP row_newbcast, so the substitution needs no barrier. One
// wave issues in order, and each step's chain (scale, broadcast, update of
// the next row of the group) is about 26 cycles of dependent latency, so
// the step's other updates (rows of later groups) are deferred by one step:
// they use the previous step's x_k and fill that wait. M streams through
// LDS in 16-column panels (panel g = the image's columns 16g .. 16g+15, 16
// KiB), three buffers deep: panel g+2 is loaded into registers while group
// g runs and written to LDS after it, behind the group's one barrier. Each
// lane reads its entries of M two steps ahead of their use. The panel in
// flight is a native vector array (Vec4): HIP's float4 struct, copied
// member-wise from memory, was kept in scratch.
template <int R>
__global__ __launch_bounds__(256) void trsm_leaf_kernel(int nb, int64_t nrhs,
                                                       const float *__restrict__ img, int rev,
                                                       float *__restrict__ Bblk, int64_t vi,
                                                       int64_t vr, float alpha) {
  constexpr int NB = kLeaf, kG = NB / 16;
  constexpr int kPanel4 = 16 * NB / 4;   // Vec4 per panel
  constexpr int kPV = kPanel4 / 256;     // Vec4 per thread per panel
  constexpr int kBufs = 3;
  __shared__ Vec4 pan_s[kBufs][kPanel4];
  __shared__ float Rd[NB];
  static_assert(NB == 256, "one reciprocal per thread");
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int j = lane & 15;
  // right-hand sides r0 .. r0 + R - 1 of this lane's row
  const int64_t r0 = ((int64_t)blockIdx.x * 16 + wave * 4 + (lane >> 4)) * R;

  // ---- every global load first: panels 0 and 1 and the reciprocals (the
  // image is 16-byte aligned: kImg is a multiple of 4 and the workspace
  // 256-byte aligned), then B
  const Vec4 *img4 = reinterpret_cast<const Vec4 *>(img);
  Vec4 p0[kPV], p1[kPV];
#pragma unroll
  for (int q = 0; q < kPV; ++q) {
    p0[q] = img4[t + 256 * q];
    p1[q] = img4[kPanel4 + t + 256 * q];
  }
  const float rdv = img[NB * NB + t];
  float x[R][kG];
#pragma unroll
  for (int h = 0; h < R; ++h) {
    const int64_t r = r0 + h < nrhs ? r0 + h : 0;
#pragma unroll
    for (int g = 0; g < kG; ++g) {
      const int i = 16 * g + j;
      x[h][g] = Bblk[(int64_t)(i < nb ? (rev ? nb - 1 - i : i) : 0) * vi + r * vr];
    }
  }
#pragma unroll
  for (int q = 0; q < kPV; ++q) {
    pan_s[0][t + 256 * q] = p0[q];
    pan_s[1][t + 256 * q] = p1[q];
  }
  Rd[t] = rdv;
#pragma unroll
  for (int h = 0; h < R; ++h)
#pragma unroll
    for (int g = 0; g < kG; ++g)
      x[h][g] = (r0 + h < nrhs && 16 * g + j < nb) ? alpha * x[h][g] : 0.f;
  __syncthreads();

  // ---- substitution
  // M(16 gg + j, k) for the lane: column k % 16 of panel k / 16
  auto m_at = [&](int k, int gg) {
    return reinterpret_cast<const float *>(pan_s[(k / 16) % kBufs])[(k % 16) * NB + 16 * gg + j];
  };
  // Entries of M are read ahead into a ring of kD steps: step k's slot is
  // k % kD, used by step k's own update of its group's rows and by step
  // k + 1's deferred updates, then refilled for step k + kD (two steps
  // ahead of its use).
  constexpr int kD = 3;
  float mb[kD][kG];
  float xd[R];  // the previous step's x_k
#pragma unroll
  for (int l = 0; l < kD; ++l)
#pragma unroll
    for (int gg = 0; gg < kG; ++gg) mb[l][gg] = m_at(l, gg);
  static_for<kG>([&](auto gc) {
    constexpr int g = decltype(gc)::value;
    Vec4 pn[kPV];  // panel g + 2, in flight during this group
    if constexpr (g + 2 < kG) {
#pragma unroll
      for (int q = 0; q < kPV; ++q) pn[q] = img4[(g + 2) * kPanel4 + t + 256 * q];
    }
    float rd[16], sg[R];  // sg: this lane's solved row 16 g + j
#pragma unroll
    for (int l = 0; l < 16; ++l) rd[l] = Rd[16 * g + l];
#pragma unroll
    for (int h = 0; h < R; ++h) sg[h] = 0.f;
    static_for<16>([&](auto lc) {
      constexpr int l = decltype(lc)::value, k = 16 * g + l;
      // Issue order, held by empty asm statements on each result (each
      // one a side effect the compiler keeps in source order): the scale
      // that starts this step's chain, two deferred updates (the DPP read
      // of the scaled value needs two wait states), the broadcast, up to
      // four more deferred updates (the broadcast's latency), the update of
      // the group's rows that ends the chain, then the remaining deferred
      // updates. The deferred updates are the previous step's, of rows in
      // later groups, with the previous step's x_k.
      constexpr int kDef = l > 0 ? (kG - 1 - g) * R : 0;
      auto deferred = [&](auto ic) {
        constexpr int i = decltype(ic)::value, gg = g + 1 + i / R, h = i % R;
        x[h][gg] = fmaf(-mb[(k - 1 + kD) % kD][gg], xd[h], x[h][gg]);
        asm volatile("" : "+v"(x[h][gg]));
      };
      float xk[R];
#pragma unroll
      for (int h = 0; h < R; ++h) {
        xk[h] = x[h][g] * rd[l];
        asm volatile("" : "+v"(xk[h]));
      }
      constexpr int kA = kDef < 2 ? kDef : 2, kB = kDef - kA < 4 ? kDef - kA : 4;
      static_for<kA>([&](auto ic) { deferred(ic); });
#pragma unroll
      for (int h = 0; h < R; ++h) {
        xk[h] = row_bcast<l>(xk[h]);
        asm volatile("" : "+v"(xk[h]));
      }
      static_for<kB>([&](auto ic) { deferred(std::integral_constant<int, kA + decltype(ic)::value>{}); });
      // this step's update of the group's rows: it feeds the next step
#pragma unroll
      for (int h = 0; h < R; ++h) {
        x[h][g] = fmaf(-mb[k % kD][g], xk[h], x[h][g]);
        asm volatile("" : "+v"(x[h][g]));
        sg[h] = j == l ? xk[h] : sg[h];
      }
      static_for<kDef - kA - kB>(
          [&](auto ic) { deferred(std::integral_constant<int, kA + kB + decltype(ic)::value>{}); });
      if constexpr (l > 0 && k - 1 + kD < NB) {
        // the previous step's slot, refilled for step k - 1 + kD
#pragma unroll
        for (int gg = (k - 1 + kD) / 16; gg < kG; ++gg) mb[(k - 1) % kD][gg] = m_at(k - 1 + kD, gg);
      }
#pragma unroll
      for (int h = 0; h < R; ++h) xd[h] = xk[h];
      __builtin_amdgcn_sched_barrier(0);
    });
    // the group's last deferred updates, then that step's slot refilled
    constexpr int kl = 16 * g + 15;
#pragma unroll
    for (int gg = g + 1; gg < kG; ++gg)
#pragma unroll
      for (int h = 0; h < R; ++h) x[h][gg] = fmaf(-mb[kl % kD][gg], xd[h], x[h][gg]);
    if constexpr (kl + kD < NB) {
#pragma unroll
      for (int gg = (kl + kD) / 16; gg < kG; ++gg) mb[kl % kD][gg] = m_at(kl + kD, gg);
    }
    // panel g + 2 into the buffer group g - 1 used; the barrier also makes it
    // visible before group g + 2 (and panel g + 1's reads ahead are already
    // covered by the previous group's barrier)
    if constexpr (g + 2 < kG) {
#pragma unroll
      for (int q = 0; q < kPV; ++q) pan_s[(g + 2) % kBufs][t + 256 * q] = pn[q];
    }
    // the group's solved rows go out now
    if (16 * g + j < nb) {
#pragma unroll
      for (int h = 0; h < R; ++h)
        if (r0 + h < nrhs) Bblk[(int64_t)(rev ? nb - 1 - (16 * g + j) : 16 * g + j) * vi + (r0 + h) * vr] = sg[h];
    }
    if constexpr (g + 1 < kG) __syncthreads();
  });
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
  float *img;  // packed diagonal blocks (trsm_pack)
};

int trsm_leaf(const Trsm &p, int64_t lo, int64_t nb, float alpha) {
  const float *img = p.img + lo / kLeaf * kImg;
  const int64_t nrhs = p.left ? p.n : p.m;
  const int rev = p.forward ? 0 : 1;
  // left: frame index = row of B (stride 1), right-hand side = column;
  // right: frame index = column of B, right-hand side = row
  float *Bblk = p.left ? p.B + lo : p.B + lo * p.ldb;
  const int64_t vi = p.left ? 1 : p.ldb, vr = p.left ? p.ldb : 1;
  // Up to 8192 right-hand sides each 16-lane row takes one (up to 2048
  // waves: two per SIMD), beyond that two (half as many LDS reads per solved
  // value). At 8192 one per row measured 26.8 against 27.0 us per leaf
  // (strsm 113.0 against 111.7 TFLOP/s).
  if (nrhs > 8192)
    trsm_leaf_kernel<2><<<(unsigned)((nrhs + 31) / 32), 256, 0, p.ctx->stream>>>(
        (int)nb, nrhs, img, rev, Bblk, vi, vr, alpha);
  else
    trsm_leaf_kernel<1><<<(unsigned)((nrhs + 15) / 16), 256, 0, p.ctx->stream>>>(
        (int)nb, nrhs, img, rev, Bblk, vi, vr, alpha);
  WGB_CHECK_LAUNCH("trsm_leaf_kernel");
  return WGB_OK;
}

// Packs every diagonal block of the solve frame into p.img (the context's
// operand workspace).
int trsm_pack(Trsm &p) {
  const int64_t order = p.left ? p.m : p.n;
  const int64_t nblk = (order + kLeaf - 1) / kLeaf;
  int st = wgb::ensure_op_workspace(p.ctx, (size_t)nblk * kImg * sizeof(float));
  if (st) return st;
  p.img = static_cast<float *>(p.ctx->op_ws);
  const bool m_is_a = p.left != p.trans;  // M is A itself, else A^T
  const int64_t mi = m_is_a ? 1 : p.lda, mk = m_is_a ? p.lda : 1;
  trsm_pack_kernel<<<dim3((unsigned)nblk, kLeaf / 16), 256, 0, p.ctx->stream>>>(
      order, p.A, p.lda, mi, mk, p.forward ? 0 : 1, p.unit, p.img);
  WGB_CHECK_LAUNCH("trsm_pack_kernel");
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
    if (!(st = trsm_pack(p))) st = trsm_solve(p, 0, p.left ? m : n, false);
  }
  if (st) return st;
  wgb::timing_end(ctx);
  return WGB_OK;
}
