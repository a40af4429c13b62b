// The level-3 routines that run on the GEMM kernel: ssyr2k, ssymm, strmm,
// strsm (wgblas src/{ssyr2k,ssymm,strmm,strsm}/*.mjs), and the native-fp64
// dsyr2k, dsymm, dtrmm (src/{dsyr2k,dsymm,dtrmm}/*.mjs) on its fp64 form.
//
// ssyr2k: one triangle GEMM launch over a two-part k range, (A, B) then
//   (B, A), when both products share a layout; else two launches, the
//   second with beta = 1.
// ssymm: the symmetric operand is expanded into a dense workspace copy
//   (LDS-tiled, coalesced both ways), then one GEMM.
// strmm: A's triangle is copied with zeros elsewhere, B is copied (the GEMM
//   cannot read and write B at once), then one GEMM whose tiles only run the
//   k-tiles the triangle reaches (about half the flops of a dense product).
// strsm: recursive halving of the triangular dimension. The diagonal blocks
//   (order <= 256) are packed once per call into the operand workspace and
//   solved by substitution inside 16-row sub-blocks (solved unknowns
//   broadcast by DPP), the updates between sub-blocks on MFMA. A solve of
//   more than one block halves down to nodes of two blocks instead: the
//   blocks' inverses are formed once (that substitution applied to the
//   identity), and one kernel per node applies the first inverse, the
//   coupling product and the second inverse on MFMA, falling back to
//   substitution per right-hand side wherever a value is not finite or a
//   block is ill-conditioned. The off-diagonal updates between diagonal
//   blocks (or nodes) are GEMMs that read the solved rows of B and write
//   other rows of B in place (disjoint memory).
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
template <typename T>
__global__ __launch_bounds__(256) void symmetrize_kernel(int64_t order, const T *__restrict__ A,
                                                         int64_t lda, int uplo,
                                                         T *__restrict__ W, int64_t ldw) {
  __shared__ T s[kTile][kTile + 1];  // s[col][row] of the source tile
  const int bi = blockIdx.x, bj = blockIdx.y;
  const bool lower = uplo == WGB_LOWER;
  const bool diag = bi == bj;
  const bool stored = lower ? bi > bj : bi < bj;
  const int si = (stored || diag) ? bi : bj, sj = (stored || diag) ? bj : bi;
  const int r = threadIdx.x & 63, ph = threadIdx.x >> 6;
  const int64_t srow = (int64_t)si * kTile + r;
  // unconditional loads from clamped addresses, all in flight together
  T v[kTile / 4];
#pragma unroll
  for (int q = 0; q < kTile / 4; ++q) {
    const int64_t scol = (int64_t)sj * kTile + ph + 4 * q;
    const bool ok = srow < order && scol < order;
    v[q] = A[(ok ? srow : 0) + (ok ? scol : 0) * lda];
  }
#pragma unroll
  for (int q = 0; q < kTile / 4; ++q) {
    const int64_t scol = (int64_t)sj * kTile + ph + 4 * q;
    s[ph + 4 * q][r] = (srow < order && scol < order) ? v[q] : (T)0;
  }
  __syncthreads();
  const int64_t row = (int64_t)bi * kTile + r;
  if (row >= order) return;
  for (int c = ph; c < kTile; c += 4) {
    const int64_t col = (int64_t)bj * kTile + c;
    if (col >= order) break;
    T v;
    if (stored)
      v = s[c][r];
    else if (!diag)
      v = s[r][c];  // W(row, col) = A(col, row), element (c, r) of tile (bj, bi)
    else
      v = (lower ? r >= c : r <= c) ? s[c][r] : s[r][c];
    W[row + col * ldw] = v;
  }
}

// trmm's side copy of its triangle's diagonal blocks (wgblas builds the
// whole triangle densely, src/shaders/triangularize.wgsl): W (same leading
// dimension as A, so the banded GEMM reads it at A's element coordinates)
// receives, inside each kSideBlock x kSideBlock diagonal block only, A's
// uplo triangle with the other triangle zeroed and, for a unit diagonal,
// ones on the diagonal. The banded GEMM reads every other block of the
// triangle in place and never reaches past a tile's diagonal block, so the
// other triangle outside the diagonal blocks is never read. Block (b, y):
// columns 8 y .. 8 y + 7 of diagonal block b, each thread 4 rows of one
// column, its loads issued before any store (one memory latency per block).
template <typename T>
__global__ __launch_bounds__(256) void diag_copy_kernel(int64_t order, const T *__restrict__ A,
                                                        int64_t lda, int uplo, int unit,
                                                        T *__restrict__ W) {
  const int64_t b0 = (int64_t)blockIdx.x * wgb::kSideBlock;
  const int64_t row0 = b0 + 4 * (threadIdx.x % 32);
  const int64_t col = b0 + 8 * blockIdx.y + threadIdx.x / 32;
  if (col >= order) return;
  const bool lower = uplo == WGB_LOWER;
  T v[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int64_t r = row0 + c;
    const bool keep = r < order && (r == col ? !unit : (lower ? r > col : r < col));
    v[c] = keep ? A[r + col * lda] : (T)0;  // the other triangle: never used, whatever A holds there
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int64_t r = row0 + c;
    if (r < order) W[r + col * lda] = (r == col && unit) ? (T)1 : v[c];
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

// strsm's diagonal blocks, packed for trsm_leaf_kernel. The solve frame
// splits into blocks of kLeaf rows (the last one nb < kLeaf rows), each
// into kSub sub-blocks of 16 rows. With N = -M (M the block in frame
// indices, zero past nb), block l's image is kImg floats at P + l kImg:
//   * pair (t, s), s < t: 256 floats at pair_at(t, s); float 4 e + c =
//     N(16 t + e % 16, 16 s + 4 (e / 16) + c) for e = 0..63, i.e. lane e's
//     B operands of the four MFMAs that update sub-block t with the
//     solved sub-block s;
//   * diagonal sub-block s: 256 floats at kDiagAt + 256 s; float 16 j + k =
//     N(16 s + j, 16 s + k) for k < j, zero for k >= j;
//   * kLeaf floats at kRdAt: 1 / M(i, i) (1 for a unit diagonal and for
//     padding rows).
// Frame element (i, k) of block l's M is Ablk[ia(i) mi + ia(k) mk], Ablk at
// A + kLeaf l (1 + lda), where ia(i) = nb-1-i for an upper system solved
// backward (rev) and i otherwise. Block (l, s) packs columns 16s .. 16s+15
// of block l through an LDS tile read with the stride-1 index fastest. The
// diagonal's reciprocals are formed once here: x * RN(1/d) is within two
// ulps of x / d, and zero, infinite and NaN diagonals give the quotient's
// special values (only a diagonal below 2^-126 in magnitude, whose
// reciprocal overflows, differs).
constexpr int kSub = kLeaf / 16, kPairs = kSub * (kSub - 1) / 2;
constexpr int kDiagAt = 256 * kPairs, kRdAt = 256 * (kPairs + kSub);
constexpr int kImg = kRdAt + (kLeaf + 63) / 64 * 64;
constexpr int kNU = kSub / 4;   // sub-blocks per wave
constexpr int kRing = 3;        // B operand slots: loaded kRing - 1 steps ahead
__host__ __device__ constexpr int pair_at(int t, int s) { return 256 * (t * (t - 1) / 2 + s); }

// The inverse of a diagonal block in the solve frame (lower triangular),
// stored as MFMA A operands: its 16 x 16 tiles (t, kb), kb <= t, each 256
// floats at inv_at(t, kb), float 4 e + c = Inv(16 t + e % 16, 16 kb +
// 4 (e / 16) + c): lane e's operands of the four 16x16x4 MFMAs that apply
// the tile, one 16-byte load. A node's coupling block -M[S, F] (below)
// uses the same tile order for all 16 x 16 tiles, at 256 (16 t + kb).
constexpr int kInvImg = 256 * (kSub * (kSub + 1) / 2);
constexpr int kCplImg = 256 * kSub * kSub;
__host__ __device__ constexpr int inv_at(int t, int kb) { return 256 * (t * (t + 1) / 2 + kb); }
// What trsm_leaf_wave does with its 16 right-hand sides: solve them in
// place, or (kLeafInvert) solve the identity's columns and write them to an
// inverse image.
enum { kLeafSolve = 0, kLeafInvert = 1 };

// NaN-propagating maximum (fmaxf drops NaN): a non-finite column sum makes
// the whole maximum non-finite.
__device__ __forceinline__ float max_nan(float a, float b) { return (b > a || b != b) ? b : a; }

// Maximum over the block's 256 threads of v (NaN-propagating); the result is
// valid in thread 0. `red` is 4 floats of LDS.
__device__ __forceinline__ float block_max_nan(float v, float *red) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v = max_nan(v, __shfl_xor(v, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return max_nan(max_nan(red[0], red[1]), max_nan(red[2], red[3]));
}

// A node's two diagonal blocks in solve order: F (solved first) and S, each
// of up to kLeaf frame rows, frame row f of a block starting at actual row
// (left) or column (right) `start` sitting at start + f (forward) or
// start + nb - 1 - f (backward).
__host__ __device__ inline int64_t node_act(int64_t start, int nb, int rev, int f) {
  return rev ? start + nb - 1 - f : start + f;
}

// Node `node`'s coupling block -M[S, F] as MFMA A operands (tile order of
// inv_at, all 16 x 16 tiles, at 256 (16 t + kb)); zero past either block's
// rows. One block packs the 16 rows 16 t .. 16 t + 15 of S through an LDS
// strip read with the stride-1 index of A fastest (trsm_pack_kernel's
// blocks past the diagonal blocks). M(i, k) = A[i mi + k mk] for actual
// indices. Nodes with one block have nothing to pack.
__device__ __forceinline__ void trsm_pack_coupling(int64_t node, int t, int64_t order,
                                                   const float *__restrict__ A, int64_t mi, int64_t mk,
                                                   int rev, float *__restrict__ C, float (*L)[kLeaf + 1]) {
  // L[i16][ff] = -M(S row 16t + i16, F row ff)
  const int tid = threadIdx.x;
  const int64_t lo = node * 2 * kLeaf;
  const int nbP = (int)(order - lo < kLeaf ? order - lo : kLeaf);
  const int64_t rest = order - lo - nbP;
  const int nbQ = (int)(rest < kLeaf ? rest : kLeaf);
  if (nbQ <= 0) return;
  const int64_t sF = rev ? lo + kLeaf : lo, sS = rev ? lo : lo + kLeaf;
  const int nbF = rev ? nbQ : nbP, nbS = rev ? nbP : nbQ;
  const bool kfast = mk == 1;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int e = tid + 256 * q;
    const int i16 = kfast ? e >> 8 : e & 15, ff = kfast ? e & 255 : e >> 4;
    const int fs = 16 * t + i16;
    const bool in = fs < nbS && ff < nbF;
    const int64_t ai = in ? node_act(sS, nbS, rev, fs) : 0, ak = in ? node_act(sF, nbF, rev, ff) : 0;
    const float v = A[ai * mi + ak * mk];
    L[i16][ff] = in ? -v : 0.f;
  }
  __syncthreads();
  float *out = C + node * kCplImg + 256 * 16 * t;
  const int e = tid, ln = e >> 2, c = e & 3;
#pragma unroll
  for (int kb = 0; kb < 16; ++kb) out[256 * kb + e] = L[ln & 15][16 * kb + 4 * (ln >> 4) + c];
}

__global__ __launch_bounds__(256) void trsm_pack_kernel(int64_t order, const float *__restrict__ A,
                                                        int64_t lda, int64_t mi, int64_t mk, int rev,
                                                        int unit, float *__restrict__ P,
                                                        float *__restrict__ slot, int64_t nblk,
                                                        float *__restrict__ cpl) {
  __shared__ float T[16][kLeaf + 1];
  if ((int64_t)blockIdx.x >= nblk) {
    // blocks past the diagonal blocks: the nodes' coupling blocks
    trsm_pack_coupling((int64_t)blockIdx.x - nblk, blockIdx.y, order, A, mi, mk, rev, cpl, T);
    return;
  }
  const int tid = threadIdx.x, s = blockIdx.y;
  const int64_t l = blockIdx.x, lo = l * kLeaf;
  const int nb = (int)(order - lo < kLeaf ? order - lo : kLeaf);
  const float *Ablk = A + lo + lo * lda;
  const bool kfast = mk == 1;  // consecutive k are adjacent in memory
  constexpr int kQ = 16 * kLeaf / 256;  // elements per thread
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
    const int e = tid + 256 * q;
    const int i = kfast ? e / 16 : e % kLeaf, kl = kfast ? e % 16 : e / kLeaf;
    const int k = 16 * s + kl;
    const bool in = i < nb && k <= i;
    const int64_t ii = in ? (rev ? nb - 1 - i : i) : 0, kk = in ? (rev ? nb - 1 - k : k) : 0;
    const float v = Ablk[ii * mi + kk * mk];
    T[kl][i] = in ? v : 0.f;  // T[kl][i] = M(i, 16 s + kl)
  }
  __syncthreads();
  float *img = P + l * kImg;
  const int e = tid >> 2, c = tid & 3;
  for (int t = s + 1; t < kSub; ++t) img[pair_at(t, s) + tid] = -T[4 * (e >> 4) + c][16 * t + (e & 15)];
  const int jj = tid >> 4, kk = tid & 15;
  img[kDiagAt + 256 * s + tid] = kk < jj ? -T[kk][16 * s + jj] : 0.f;
  if (tid < 16) {
    const int k = 16 * s + tid;
    img[kRdAt + k] = 1.f / ((unit || k >= nb) ? 1.f : T[tid][k]);
  }
  if (slot) {
    // the largest column sum of |M| over this block's 16 columns (a unit
    // diagonal counted as 1): slot[l * 32 + s], for the inverse path's
    // condition estimate
    const int kl = tid >> 4, part = tid & 15, k = 16 * s + kl;
    float sum = 0.f;
    for (int i = part; i < kLeaf; i += 16) sum += (i == k && unit && k < nb) ? 1.f : fabsf(T[kl][i]);
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) sum += __shfl_xor(sum, o);
    __shared__ float red[4];
    const float m = block_max_nan(sum, red);
    if (tid == 0) slot[l * 32 + s] = m;
  }
}

// The solved sub-block handed between waves, [row k][right-hand side], rows
// 20 floats apart: both the 16-byte stores of the solving wave and the
// column reads of the MFMA A operand are free of bank conflicts.
constexpr int kXs = 20;

// One substitution step for four right-hand sides: x = acc * rd in every
// lane, then acc += md * (x of lane K of the 16-lane row): v_fmac_f32 with a
// DPP row_newbcast source, the broadcast and the update in one instruction.
// Each DPP source is written four instructions before it is read (the
// hardware needs two wait states between a VALU write and a DPP read).
template <int K>
__device__ __forceinline__ void subst_step(Vec4 &acc, float rd, float md) {
  float a0 = acc[0], a1 = acc[1], a2 = acc[2], a3 = acc[3], t0, t1, t2, t3;
  asm volatile(
      "v_mul_f32 %4, %8, %0\n\t"
      "v_mul_f32 %5, %8, %1\n\t"
      "v_mul_f32 %6, %8, %2\n\t"
      "v_mul_f32 %7, %8, %3\n\t"
      "v_fmac_f32_dpp %0, %4, %9 row_newbcast:%10 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %5, %9 row_newbcast:%10 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %2, %6, %9 row_newbcast:%10 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %3, %7, %9 row_newbcast:%10 row_mask:0xf bank_mask:0xf"
      : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3)
      : "s"(rd), "v"(md), "n"(K));
  acc = Vec4{a0, a1, a2, a3};
}

// acc += sum over c of the 16x16x4 products (a[c], b[c]): one 16 x 16 x 16
// update.
__device__ __forceinline__ Vec4 mfma4(Vec4 acc, const float (&a)[4], Vec4 b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], acc, 0, 0, 0);
  return acc;
}

// Substitution solve of one diagonal block, in the solve frame: for 16
// right-hand sides v, M x = alpha v with M lower triangular of order
// nb <= kLeaf, given as its image `img` (trsm_pack_kernel). Element i of
// right-hand side r is Bblk[ia(i) vi + r vr], where ia(i) = nb-1-i for an
// upper system solved backward (rev) and i otherwise; the solution
// overwrites v.
//
// The block's kSub sub-blocks of 16 rows are dealt to its 4 waves: the wave
// playing part w (W, trsm_leaf_kernel) owns sub-blocks t = 4u + w
// (u = 0 .. kNU-1) and holds each as a 16x16x4
// MFMA accumulator of (right-hand side) x (row): lane j + 16 q holds row
// 16 t + j of right-hand sides 4q .. 4q+3. Step s (s = 0 .. kSub-1):
//   * the owner of sub-block s solves it by substitution, in the
//     column-oriented order of wgblas's strsm_small.wgsl and of reference
//     BLAS: x_k = x_k * (1 / M(k,k)), broadcast from lane k by DPP
//     row_newbcast, and every lane subtracts M(16s + j, 16s + k) x_k from
//     its row (one v_fmac_f32 with the DPP source). Rows j <= k are
//     multiplied by the image's zeros there and keep their value while
//     every x_k is finite, so each lane's solution is its row times the
//     reciprocal once more at the end. A wave that saw a non-finite value
//     redoes the sub-block from its saved rows, keeping each row's x_k as it
//     is broadcast: IEEE specials land where substitution puts them. The
//     solved rows go to LDS (Xs) and out to B;
//   * barrier; every wave updates its sub-blocks t > s with them: four MFMAs
//     whose A operand is the solved rows (from Xs) and B operand the pair
//     (t, s) of the image, read from global memory (written kRing - 1
//     steps ahead; the scheduler issues them at the end of the previous
//     step, and holding them at the earlier point measured slower). The
//     owner of sub-block s+1 updates that one first and defers its others
//     into its substitution (one MFMA per substitution step at kLeaf 256,
//     up to two for larger blocks), so the next step's substitution starts
//     right after the four MFMAs it needs.
// The step loop is unrolled with s and the wave's part w known at compile
// time (register arrays need constant indices), one copy per part. Making w
// a uniform runtime branch instead (one copy of the code for all four) held
// more registers and measured slower (18.1 against 16.2 us per leaf at 4096
// right-hand sides).
// The off-diagonal products are summed by the MFMA (four per instruction)
// rather than one subtraction at a time; within a sub-block the order is
// that of substitution. alpha is applied as v is read. Rows past nb are
// padding with a unit diagonal and zero right-hand side; they never feed
// real rows.
template <int W, int MODE = kLeafSolve>
__device__ __forceinline__ void trsm_leaf_wave(int nb, int64_t nrhs, const float *__restrict__ img,
                                               int rev, float *__restrict__ Bblk, int64_t vi,
                                               int64_t vr, float alpha, int64_t r0, int lane,
                                               float (*__restrict__ Xs)[16][kXs],
                                               uint32_t store_mask = 0xffffu,
                                               float *__restrict__ inv = nullptr,
                                               Vec4 *csum = nullptr) {
  const int j = lane & 15, q = lane >> 4;
  const Vec4 *img4 = reinterpret_cast<const Vec4 *>(img);
  const float *rdp = img + kRdAt;
  auto frame = [&](int i) -> int64_t { return rev ? nb - 1 - i : i; };
  auto rhs_ok = [&](int v) { return r0 + 4 * q + v < nrhs; };

  // ---- global loads: this wave's rows of the right-hand sides, the B
  // operands of the first steps, the first diagonal sub-block it solves
  Vec4 acc[kNU];
  static_for<kNU>([&](auto uc) {
    constexpr int u = decltype(uc)::value;
    const int i = 16 * (4 * u + W) + j;
    const int64_t ii = i < nb ? frame(i) : 0;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if constexpr (MODE == kLeafInvert)
        acc[u][v] = i == (int)r0 + 4 * q + v ? 1.f : 0.f;  // column r0 + 4q + v of the identity
      else
        acc[u][v] = Bblk[ii * vi + (rhs_ok(v) ? r0 + 4 * q + v : 0) * vr];
    }
  });
  // B operands of step s's update of sub-block 4u + w: slot s % kRing
  Vec4 bop[kRing][kNU];
  static_for<kRing - 1>([&](auto sc) {
    constexpr int s = decltype(sc)::value;
    static_for<kNU>([&](auto uc) {
      constexpr int u = decltype(uc)::value;
      if constexpr (4 * u + W > s) bop[s][u] = img4[pair_at(4 * u + W, s) / 4 + lane];
    });
  });
  Vec4 md4[4];    // row j of the next diagonal sub-block this wave solves,
  float rdj;      // that row's reciprocal
  float rdn[16];  // and the sub-block's reciprocals (uniform)
#pragma unroll
  for (int m = 0; m < 4; ++m) md4[m] = img4[(kDiagAt + 256 * W + 16 * j) / 4 + m];
  rdj = rdp[16 * W + j];
#pragma unroll
  for (int k = 0; k < 16; ++k) rdn[k] = rdp[16 * W + k];
  static_for<kNU>([&](auto uc) {
    constexpr int u = decltype(uc)::value;
    const bool row_ok = 16 * (4 * u + W) + j < nb;
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[u][v] = (row_ok && rhs_ok(v)) ? alpha * acc[u][v] : 0.f;
  });

  float apend[4];  // a deferred update: solved rows and B operands
  Vec4 bpend[kNU];
  static_for<kSub>([&](auto sc) {
    constexpr int s = decltype(sc)::value, us = s / 4;
    Vec4 x;  // this lane's solved row of sub-block s (owner)
    if constexpr (s % 4 == W) {
      // deferred MFMAs of the previous step: sub-blocks u > us
      constexpr int kPend = s > 0 ? 4 * (kNU - 1 - us) : 0;
      const Vec4 keep = acc[us];
      float rds[16], md[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        rds[k] = rdn[k];
        md[k] = md4[k / 4][k % 4];
      }
      static_for<16>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        static_for<2>([&](auto hc) {
          constexpr int i = k + 16 * decltype(hc)::value;
          if constexpr (i < kPend) {
            constexpr int u = us + 1 + i / 4, c = i % 4;
            acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(apend[c], bpend[u][c], acc[u], 0, 0, 0);
          }
        });
        subst_step<k>(acc[us], rds[k], md[k]);
        __builtin_amdgcn_sched_barrier(0);
      });
      bool bad = false;
#pragma unroll
      for (int v = 0; v < 4; ++v) bad |= !__builtin_isfinite(acc[us][v]);
      if (__ballot(bad)) {
        // a non-finite value: substitution again, each row kept as solved
        acc[us] = keep;
        x = Vec4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
        for (int k = 0; k < 16; ++k) {
          const Vec4 xk = acc[us] * rdp[16 * s + k];
          const float mk = img[kDiagAt + 256 * s + 16 * j + k];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            x[v] = j == k ? xk[v] : x[v];
            acc[us][v] = fmaf(mk, __shfl(xk[v], (lane & 48) | k), acc[us][v]);
          }
        }
      } else {
        x = acc[us] * rdj;
      }
      *reinterpret_cast<Vec4 *>(&Xs[s & 1][j][4 * q]) = x;
      if constexpr (s + 4 < kSub) {
#pragma unroll
        for (int m = 0; m < 4; ++m) md4[m] = img4[(kDiagAt + 256 * (s + 4) + 16 * j) / 4 + m];
        rdj = rdp[16 * (s + 4) + j];
#pragma unroll
        for (int k = 0; k < 16; ++k) rdn[k] = rdp[16 * (s + 4) + k];
      }
    }
    __syncthreads();
    if constexpr (s + 1 < kSub) {
      float a[4];  // A operand: solved row 4q + c of right-hand side j
#pragma unroll
      for (int c = 0; c < 4; ++c) a[c] = Xs[s & 1][4 * q + c][j];
      constexpr int sa = s + kRing - 1;  // the step whose operands load now
      if constexpr (sa < kSub) {
        static_for<kNU>([&](auto uc) {
          constexpr int u = decltype(uc)::value;
          if constexpr (4 * u + W > sa) bop[sa % kRing][u] = img4[pair_at(4 * u + W, sa) / 4 + lane];
        });
      }
      Vec4(&bcur)[kNU] = bop[s % kRing];
      if constexpr ((s + 1) % 4 == W) {
        constexpr int un = (s + 1) / 4;
        acc[un] = mfma4(acc[un], a, bcur[un]);
#pragma unroll
        for (int c = 0; c < 4; ++c) apend[c] = a[c];
        static_for<kNU>([&](auto uc) {
          constexpr int u = decltype(uc)::value;
          if constexpr (u > un) bpend[u] = bcur[u];
        });
      } else {
        static_for<kNU>([&](auto uc) {
          constexpr int u = decltype(uc)::value;
          if constexpr (4 * u + W > s) acc[u] = mfma4(acc[u], a, bcur[u]);
        });
      }
    }
    if constexpr (s % 4 == W) {
      const int i = 16 * s + j;
      if constexpr (MODE == kLeafInvert) {
        // rows 16s .. 16s+15 of inverse columns r0 .. r0+15: tile (s, r0 / 16)
        // of the inverse image, this lane's four values in one 16-byte store
        // (padding rows and columns are exact zeros; tiles right of the
        // diagonal are never read and not written)
        const int kb = (int)(r0 >> 4);
        if (kb <= s) *reinterpret_cast<Vec4 *>(inv + inv_at(s, kb) + 4 * lane) = x;
#pragma unroll
        for (int v = 0; v < 4; ++v) (*csum)[v] += fabsf(x[v]);
      } else if (i < nb) {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (rhs_ok(v) && ((store_mask >> (4 * q + v)) & 1u)) Bblk[frame(i) * vi + (r0 + 4 * q + v) * vr] = x[v];
      }
    }
  });
}

// One block per 16 right-hand sides; wave w plays part w. (Rotating the
// parts by block parity, so that two blocks sharing a compute unit
// substitute on different SIMDs, measured no different.)
__global__ __launch_bounds__(256) void trsm_leaf_kernel(int nb, int64_t nrhs,
                                                       const float *__restrict__ img, int rev,
                                                       float *__restrict__ Bblk, int64_t vi,
                                                       int64_t vr, float alpha) {
  __shared__ float Xs[2][16][kXs];
  const int lane = threadIdx.x & 63;
  const int part = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t r0 = (int64_t)blockIdx.x * 16;
  switch (part) {
    case 0: trsm_leaf_wave<0>(nb, nrhs, img, rev, Bblk, vi, vr, alpha, r0, lane, Xs); break;
    case 1: trsm_leaf_wave<1>(nb, nrhs, img, rev, Bblk, vi, vr, alpha, r0, lane, Xs); break;
    case 2: trsm_leaf_wave<2>(nb, nrhs, img, rev, Bblk, vi, vr, alpha, r0, lane, Xs); break;
    default: trsm_leaf_wave<3>(nb, nrhs, img, rev, Bblk, vi, vr, alpha, r0, lane, Xs); break;
  }
}

// Inverse of every diagonal block in the solve frame, written as an inverse
// image (inv_at): block (g, l) solves M_l x = e_r for the identity's columns
// r = 16 g .. 16 g + 15 with the substitution above, so the inverse is
// substitution's to the last bit in every column. Each block also records
// the largest column sum of |inverse| over its 16 columns in slot[l * 32 +
// 16 + g] (non-finite when any entry is), for the condition estimate.
__global__ __launch_bounds__(256) void trsm_invert_kernel(int64_t order, const float *__restrict__ img,
                                                         float *__restrict__ inv,
                                                         float *__restrict__ slot) {
  __shared__ float Xs[2][16][kXs];
  __shared__ float red[4];
  const int lane = threadIdx.x & 63;
  const int part = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t l = blockIdx.y, lo = l * kLeaf;
  const int nb = (int)(order - lo < kLeaf ? order - lo : kLeaf);
  const int64_t r0 = (int64_t)blockIdx.x * 16;
  const float *im = img + l * kImg;
  float *iv = inv + l * kInvImg;
  Vec4 cs = Vec4{0.f, 0.f, 0.f, 0.f};
  switch (part) {
    case 0: trsm_leaf_wave<0, kLeafInvert>(nb, kLeaf, im, 0, nullptr, 0, 0, 1.f, r0, lane, Xs, 0, iv, &cs); break;
    case 1: trsm_leaf_wave<1, kLeafInvert>(nb, kLeaf, im, 0, nullptr, 0, 0, 1.f, r0, lane, Xs, 0, iv, &cs); break;
    case 2: trsm_leaf_wave<2, kLeafInvert>(nb, kLeaf, im, 0, nullptr, 0, 0, 1.f, r0, lane, Xs, 0, iv, &cs); break;
    default: trsm_leaf_wave<3, kLeafInvert>(nb, kLeaf, im, 0, nullptr, 0, 0, 1.f, r0, lane, Xs, 0, iv, &cs); break;
  }
  // lane j + 16 q holds partial sums of columns 4q .. 4q+3 over its rows:
  // add the 16 lanes of each q, then the four waves
  __shared__ float colsum[4][16];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    float c = cs[v];
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) c += __shfl_xor(c, o);
    if ((lane & 15) == 0) colsum[part][4 * (lane >> 4) + v] = c;
  }
  __syncthreads();
  float m = 0.f;
  if (threadIdx.x < 16) m = colsum[0][threadIdx.x] + colsum[1][threadIdx.x] + colsum[2][threadIdx.x] +
                           colsum[3][threadIdx.x];
  m = block_max_nan(m, red);
  if (threadIdx.x == 0) slot[l * 32 + 16 + blockIdx.x] = m;
}

// One 512-row node of the solve frame: F's rows, then S's, for 16
// right-hand sides per block (4 waves).
struct NodeArgs {
  int nbF, nbS;  // rows of F and S (nbS == 0: F alone)
  int rev;
  int64_t nrhs, vi, vr;
  float *BF, *BS;  // element (frame f, right-hand side r) at B_[act(f) vi + r vr]
  float alpha;     // applied to B as it is read
  const float *imgF, *imgS;    // substitution images (trsm_pack_kernel)
  const float *invF, *invS;    // inverse images (trsm_invert_kernel)
  const float *cpl;            // -M[S, F] (trsm_pack_coupling_kernel)
  const float *slotF, *slotS;  // column-sum maxima of M and of its inverse
};

// Right-hand sides r0 .. r0+15 of F (and S, when nbS > 0) into panels P[0]
// (P[1]) as [r][f], times alphaF (alphaS), zero past nb or nrhs; bit r of bad[0]
// (bad[1]) set for a non-finite value. Every load is issued before the first
// one is used (no branch between them: 32 in flight per thread), frame rows
// fastest when they are adjacent in memory (left side), right-hand sides
// fastest otherwise.
__device__ __forceinline__ void node_load_panels(const float *__restrict__ BF, int nbF,
                                                 const float *__restrict__ BS, int nbS, int rev,
                                                 int64_t vi, int64_t vr, int64_t r0, int64_t nrhs,
                                                 float alphaF, float alphaS, float (*P)[16][kLeaf + 4],
                                                 uint32_t *bad) {
  const int tid = threadIdx.x;
  const bool ffast = vi == 1;
  // element q of this thread: frame row f0 + fs q of right-hand side
  // r0 + rr0 + rs q, at base + q step (or nowhere when out of range)
  const int f0 = ffast ? tid & 255 : tid >> 4, fs = ffast ? 0 : 16;
  const int rr0 = ffast ? 0 : tid & 15, rs = ffast ? 1 : 0;
  float v[2][16];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const float *B = b ? BS : BF;
    const int nb = b ? nbS : nbF;
    const int64_t fstep = rev ? -vi : vi;  // memory step of frame row f + 1
    const float *base = B + (rev ? nb - 1 - f0 : f0) * vi + (r0 + rr0) * vr;
    const int64_t step = ffast ? vr : 16 * fstep;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const bool in = f0 + fs * q < nb && r0 + rr0 + rs * q < nrhs;
      v[b][q] = *(in ? base + q * step : B);
    }
  }
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int nb = b ? nbS : nbF;
    const float alpha = b ? alphaS : alphaF;
    uint32_t mask = 0u;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int f = f0 + fs * q, r = rr0 + rs * q;
      const float x = (f < nb && r0 + r < nrhs) ? alpha * v[b][q] : 0.f;
      P[b][r][f] = x;
      mask |= __builtin_isfinite(x) ? 0u : 1u << r;
    }
    if (mask) atomicOr(&bad[b], mask);
  }
}

// Row block (16 frame rows) u = 0..3 of wave W in the node kernel: W,
// 7 - W, 8 + W, 15 - W, so every wave applies 34 of an inverse's 136
// tiles (row block t has t + 1 of them).
__host__ __device__ constexpr int node_rb(int u, int W) {
  return u == 0 ? W : u == 1 ? 7 - W : u == 2 ? 8 + W : 15 - W;
}

// x[u] into panel rows 16 t + 4 g .. + 3 (t = node_rb(u, W)) of right-hand
// side i16.
template <int W>
__device__ __forceinline__ void node_to_panel(const Vec4 (&x)[4], float (*panel)[kLeaf + 4], int lane) {
  const int g = lane >> 4, i16 = lane & 15;
#pragma unroll
  for (int u = 0; u < 4; ++u) *reinterpret_cast<Vec4 *>(&panel[i16][16 * node_rb(u, W) + 4 * g]) = x[u];
}

// Bit i16 of *bad for any non-finite value among this lane's x.
__device__ __forceinline__ void node_flag(const Vec4 (&x)[4], int lane, uint32_t *bad) {
  bool b = false;
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int c = 0; c < 4; ++c) b |= !__builtin_isfinite(x[u][c]);
  if (b) atomicOr(bad, 1u << (lane & 15));
}

// Stores x's rows below nb to B for the right-hand sides whose bit in
// `skip` is clear.
template <int W>
__device__ __forceinline__ void node_store(const Vec4 (&x)[4], float *__restrict__ B, int nb, int rev,
                                           int64_t vi, int64_t vr, int64_t r0, int64_t nrhs,
                                           uint32_t skip, int lane) {
  const int g = lane >> 4, i16 = lane & 15;
  if (r0 + i16 >= nrhs || ((skip >> i16) & 1u)) return;
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int f = 16 * node_rb(u, W) + 4 * g + c;
      if (f < nb) B[node_act(0, nb, rev, f) * vi + (r0 + i16) * vr] = x[u][c];
    }
}

// panel[r][f] (rows below nb, right-hand sides below nrhs) to B, all 256
// threads, in node_load_panel's order (consecutive threads write adjacent
// elements): the fast path's stores. The MFMA layout itself gives each lane
// one right-hand side, which would scatter every store instruction over 16
// columns.
__device__ __forceinline__ void node_store_panel(const float (*panel)[kLeaf + 4], float *__restrict__ B,
                                                 int nb, int rev, int64_t vi, int64_t vr, int64_t r0,
                                                 int64_t nrhs) {
  const int tid = threadIdx.x;
  const bool ffast = vi == 1;
#pragma unroll 4
  for (int q = 0; q < 16; ++q) {
    const int e = tid + 256 * q;
    const int f = ffast ? e & 255 : e >> 4, r = ffast ? e >> 8 : e & 15;
    if (f < nb && r0 + r < nrhs) B[node_act(0, nb, rev, f) * vi + (r0 + r) * vr] = panel[r][f];
  }
}

// Whether an inverse image may stand for substitution: finite, and the
// 1-norm condition estimate ||M||_1 ||M^-1||_1 at most kCondMax (above it
// the inverse's rounding, amplified by the condition number, could exceed
// substitution's backward error).
constexpr float kCondMax = 16.f;
__device__ __forceinline__ bool node_usable(const float *__restrict__ slot) {
  float m = 0.f, v = 0.f;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    m = max_nan(m, slot[k]);
    v = max_nan(v, slot[16 + k]);
  }
  return m * v <= kCondMax;
}

// The fast path's products for wave W (row blocks node_rb(u, W)) as one
// stream of NS = 16 (F alone) or 48 k-tile steps: X_F = inv_F P[0] (steps 0-15), T = P[1] - M[S, F] X_F
// (16-31), X_S = inv_S T (32-47), with the panel hand-offs between them.
// Each step's A operands are loaded kAhead steps before it (a register
// ring), across the phase boundaries too: one wave per SIMD leaves the
// loads' latency to be covered that way. Every accumulator sees the same
// MFMA sequence (k-tiles ascending, four MFMAs each, row blocks
// interleaved) as node_recompute, so the results are the same bits.
// `pre` (the panels' loads and a barrier) runs once the first steps' operand
// loads are issued. Non-finite values set bit i16 of flag[0] (X_F), flag[1]
// (T) or flag[2] (X_S). On return X_F is in P[0] and X_S in P[1] too
// (complete after the caller's next barrier).
constexpr int kAhead = 3;
template <int W, bool TWO, typename Pre>
__device__ __forceinline__ void node_stream(const NodeArgs &a, int lane, float (*P)[16][kLeaf + 4],
                                            uint32_t *flag, Vec4 (&xf)[4], Vec4 (&xt)[4],
                                            Vec4 (&xs)[4], Pre &&pre) {
  constexpr int NS = TWO ? 3 * kSub : kSub;
  const int g = lane >> 4, i16 = lane & 15;
  const Vec4 *ivF = reinterpret_cast<const Vec4 *>(a.invF);
  const Vec4 *ivS = reinterpret_cast<const Vec4 *>(a.invS);
  const Vec4 *cp = reinterpret_cast<const Vec4 *>(a.cpl);
  Vec4 ring[kAhead + 1][4];
  Vec4 bcur;
  // whether step s has a tile for row block u, and the load of it
  auto issue = [&](auto sc) {
    constexpr int st = decltype(sc)::value, ph = st / kSub, kb = st % kSub, slot = st % (kAhead + 1);
    static_for<4>([&](auto uc) {
      constexpr int u = decltype(uc)::value, t = node_rb(u, W);
      if constexpr (ph == 0 && t >= kb) ring[slot][u] = ivF[inv_at(t, kb) / 4 + lane];
      if constexpr (ph == 1) ring[slot][u] = cp[64 * (16 * t + kb) + lane];
      if constexpr (ph == 2 && t >= kb) ring[slot][u] = ivS[inv_at(t, kb) / 4 + lane];
    });
  };
  static_for<kAhead>(issue);
  pre();  // the panels' loads, in flight with the first steps' operand loads
#pragma unroll
  for (int u = 0; u < 4; ++u) xf[u] = Vec4{0.f, 0.f, 0.f, 0.f};
  static_for<NS>([&](auto sc) {
    constexpr int st = decltype(sc)::value, ph = st / kSub, kb = st % kSub;
    constexpr int slot = st % (kAhead + 1);
    // fences keep each step's loads where they are issued (the scheduler
    // would otherwise hoist them all and run out of registers)
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (st + kAhead < NS) issue(std::integral_constant<int, st + kAhead>{});
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (ph == 1 && kb == 0) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        xt[u] = *reinterpret_cast<const Vec4 *>(&P[1][i16][16 * node_rb(u, W) + 4 * g]);
    }
    if constexpr (ph == 2 && kb == 0) {
#pragma unroll
      for (int u = 0; u < 4; ++u) xs[u] = Vec4{0.f, 0.f, 0.f, 0.f};
    }
    Vec4(&acc)[4] = ph == 0 ? xf : ph == 1 ? xt : xs;
    const float(*src)[kLeaf + 4] = ph == 2 ? P[1] : P[0];
    // B operands: this step's were read one step earlier (inside a phase;
    // a phase's first step reads its own, after the hand-off barriers)
    if constexpr (kb == 0) bcur = *reinterpret_cast<const Vec4 *>(&src[i16][4 * g]);
    Vec4 bnext;
    if constexpr (kb + 1 < kSub) bnext = *reinterpret_cast<const Vec4 *>(&src[i16][16 * (kb + 1) + 4 * g]);
    const Vec4 b4 = bcur;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      static_for<4>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        if constexpr (ph == 1 || node_rb(u, W) >= kb)
          acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(ring[slot][u][c], b4[c], acc[u], 0, 0, 0);
      });
    if constexpr (kb + 1 < kSub) bcur = bnext;
    if constexpr (kb == kSub - 1 && ph == 0) {
      node_flag(xf, lane, &flag[0]);
      __syncthreads();  // every wave has read B_F's panel
      node_to_panel<W>(xf, P[0], lane);
      if constexpr (TWO) __syncthreads();  // X_F complete in P[0]
    }
    if constexpr (kb == kSub - 1 && ph == 1) {
      node_flag(xt, lane, &flag[1]);
      __syncthreads();  // every wave has read S's right-hand sides and X_F
      node_to_panel<W>(xt, P[1], lane);
      __syncthreads();  // T complete in P[1]
    }
    if constexpr (kb == kSub - 1 && ph == 2) {
      node_flag(xs, lane, &flag[2]);
      __syncthreads();  // every wave has read T
      node_to_panel<W>(xs, P[1], lane);
    }
  });
}

// node_stream's T and X_S steps again, as runtime loops (the slow path's
// copy: little code, few registers), with the same MFMA sequence per
// accumulator, so the same bits. X_F is in P[0], S's right-hand sides in
// P[1]; flag[1] / flag[2] as in node_stream.
template <int W>
__device__ __forceinline__ void node_recompute(const NodeArgs &a, int lane, float (*P)[16][kLeaf + 4],
                                               uint32_t *flag, Vec4 (&xt)[4], Vec4 (&xs)[4]) {
  const int g = lane >> 4, i16 = lane & 15;
  const Vec4 *cp = reinterpret_cast<const Vec4 *>(a.cpl);
  const Vec4 *iv = reinterpret_cast<const Vec4 *>(a.invS);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    xt[u] = *reinterpret_cast<const Vec4 *>(&P[1][i16][16 * node_rb(u, W) + 4 * g]);
    xs[u] = Vec4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll 1
  for (int kb = 0; kb < kSub; ++kb) {
    Vec4 a4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) a4[u] = cp[64 * (16 * node_rb(u, W) + kb) + lane];
    const Vec4 b4 = *reinterpret_cast<const Vec4 *>(&P[0][i16][16 * kb + 4 * g]);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int u = 0; u < 4; ++u) xt[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[u][c], b4[c], xt[u], 0, 0, 0);
  }
  node_flag(xt, lane, &flag[1]);
  __syncthreads();  // every wave has read S's right-hand sides and X_F
  node_to_panel<W>(xt, P[1], lane);
  __syncthreads();  // T complete in P[1]
#pragma unroll 1
  for (int kb = 0; kb < kSub; ++kb) {
    Vec4 a4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (node_rb(u, W) >= kb) a4[u] = iv[inv_at(node_rb(u, W), kb) / 4 + lane];
    const Vec4 b4 = *reinterpret_cast<const Vec4 *>(&P[1][i16][16 * kb + 4 * g]);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (node_rb(u, W) >= kb) xs[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[u][c], b4[c], xs[u], 0, 0, 0);
  }
  node_flag(xs, lane, &flag[2]);
}

// The node's wave W. Fast path (every value finite, both inverses usable):
// X_F = inv_F (alpha B_F), T = alpha B_S - M[S, F] X_F, X_S = inv_S T, all in
// registers and LDS, then both stored. Otherwise, per right-hand side: one
// that met a non-finite value in a block, or a block whose inverse is not
// usable, takes substitution (trsm_leaf_wave) in that block, exactly where
// the substitution-only solve would: a right-hand side's bits do not depend
// on the other right-hand sides, and Inf / NaN land where substitution puts
// them (the coupling product's IEEE specials do not depend on its order).
template <int W, bool TWO>
__device__ __forceinline__ void trsm_node_wave(const NodeArgs &a, int64_t r0, int lane,
                                               float (*P)[16][kLeaf + 4], float (*Xs)[16][kXs],
                                               uint32_t *bad) {
  constexpr bool two = TWO;
  const bool useF = node_usable(a.slotF), useS = two && node_usable(a.slotS);
  Vec4 xf[4], xt[4], xs[4];
  node_stream<W, TWO>(a, lane, P, bad, xf, xt, xs, [&] {
    node_load_panels(a.BF, a.nbF, a.BS, a.nbS, a.rev, a.vi, a.vr, r0, a.nrhs, a.alpha, a.alpha, P, bad);
    __syncthreads();  // both panels in LDS
  });
  __syncthreads();  // every flag set
  const uint32_t all = 0xffffu;
  const uint32_t pF = useF ? bad[0] : all;
  const uint32_t pS = two ? (useS ? (bad[1] | bad[2]) : all) : 0u;
  if ((pF | pS) == 0u) {
    node_store_panel(P[0], a.BF, a.nbF, a.rev, a.vi, a.vr, r0, a.nrhs);
    if (two) node_store_panel(P[1], a.BS, a.nbS, a.rev, a.vi, a.vr, r0, a.nrhs);
    return;
  }
  // Substitution for F's marked right-hand sides (reading B_F, untouched so
  // far), then the inverse's results for the others.
  if (pF) trsm_leaf_wave<W>(a.nbF, a.nrhs, a.imgF, a.rev, a.BF, a.vi, a.vr, a.alpha, r0, lane, Xs, pF);
  node_store<W>(xf, a.BF, a.nbF, a.rev, a.vi, a.vr, r0, a.nrhs, pF, lane);
  if (!two) return;
  __syncthreads();  // X_F in B for every right-hand side
  uint32_t qS = pS;
  if (pF) {
    // X_F changed for the marked right-hand sides: T again from B (the
    // same operands and order, so the same bits for the others)
    // X_F (times 1: the same values) and S's right-hand sides again; the
    // flags of X_F's reload are not needed (bad[4]), S's go to bad[5]
    node_load_panels(a.BF, a.nbF, a.BS, a.nbS, a.rev, a.vi, a.vr, r0, a.nrhs, 1.f, a.alpha, P, &bad[4]);
    __syncthreads();
    node_recompute<W>(a, lane, P, &bad[4], xt, xs);  // T: bad[5], X_S: bad[6]
    __syncthreads();
    qS = useS ? (bad[5] | bad[6]) : all;
  }
  // T into S's rows for substitution's marked right-hand sides, which read it
  // from B; then the inverse's results for the others
  node_store<W>(xt, a.BS, a.nbS, a.rev, a.vi, a.vr, r0, a.nrhs, ~qS, lane);
  __syncthreads();
  if (qS) trsm_leaf_wave<W>(a.nbS, a.nrhs, a.imgS, a.rev, a.BS, a.vi, a.vr, 1.f, r0, lane, Xs, qS);
  node_store<W>(xs, a.BS, a.nbS, a.rev, a.vi, a.vr, r0, a.nrhs, qS, lane);
}

__global__ __launch_bounds__(256) void trsm_node_kernel(NodeArgs a) {
  __shared__ float P[2][16][kLeaf + 4];  // [block][right-hand side][frame row]
  __shared__ float Xs[2][16][kXs];
  __shared__ uint32_t bad[8];
  const int lane = threadIdx.x & 63;
  const int part = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t r0 = (int64_t)blockIdx.x * 16;
  if (threadIdx.x < 8) bad[threadIdx.x] = 0u;
  __syncthreads();
  if (a.nbS > 0) {
    switch (part) {
      case 0: trsm_node_wave<0, true>(a, r0, lane, P, Xs, bad); break;
      case 1: trsm_node_wave<1, true>(a, r0, lane, P, Xs, bad); break;
      case 2: trsm_node_wave<2, true>(a, r0, lane, P, Xs, bad); break;
      default: trsm_node_wave<3, true>(a, r0, lane, P, Xs, bad); break;
    }
  } else {
    switch (part) {
      case 0: trsm_node_wave<0, false>(a, r0, lane, P, Xs, bad); break;
      case 1: trsm_node_wave<1, false>(a, r0, lane, P, Xs, bad); break;
      case 2: trsm_node_wave<2, false>(a, r0, lane, P, Xs, bad); break;
      default: trsm_node_wave<3, false>(a, r0, lane, P, Xs, bad); break;
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
  float *img;  // packed diagonal blocks (trsm_pack)
  // The node path (solve order above one block): the diagonal blocks'
  // inverses, the nodes' coupling blocks, and 32 column-sum maxima per block
  // (16 of M, 16 of its inverse); null otherwise.
  bool nodes = false;
  float *inv = nullptr, *cpl = nullptr, *slot = nullptr;
};

constexpr int kNode = 2 * kLeaf;  // rows one trsm_node_kernel launch solves

int trsm_leaf(const Trsm &p, int64_t lo, int64_t nb, float alpha) {
  const float *img = p.img + lo / kLeaf * kImg;
  const int64_t nrhs = p.left ? p.n : p.m;
  const int rev = p.forward ? 0 : 1;
  // left: frame index = row of B (stride 1), right-hand side = column;
  // right: frame index = column of B, right-hand side = row
  float *Bblk = p.left ? p.B + lo : p.B + lo * p.ldb;
  const int64_t vi = p.left ? 1 : p.ldb, vr = p.left ? p.ldb : 1;
  trsm_leaf_kernel<<<(unsigned)((nrhs + 15) / 16), 256, 0, p.ctx->stream>>>(
      (int)nb, nrhs, img, rev, Bblk, vi, vr, alpha);
  WGB_CHECK_LAUNCH("trsm_leaf_kernel");
  return WGB_OK;
}

// Packs every diagonal block of the solve frame into p.img (the context's
// operand workspace). With more than one block (the node path) also: each
// block's inverse (trsm_invert_kernel, substitution on the identity), each
// node's coupling block, and the column sums for the condition estimates.
int trsm_pack(Trsm &p) {
  const int64_t order = p.left ? p.m : p.n;
  const int64_t nblk = (order + kLeaf - 1) / kLeaf;
  const int64_t nnode = (order + kNode - 1) / kNode;
  p.nodes = order > kLeaf;
  size_t floats = (size_t)nblk * kImg;
  if (p.nodes) floats += (size_t)nblk * kInvImg + (size_t)nnode * kCplImg + (size_t)nblk * 32;
  int st = wgb::ensure_op_workspace(p.ctx, floats * sizeof(float));
  if (st) return st;
  p.img = static_cast<float *>(p.ctx->op_ws);
  if (p.nodes) {
    p.inv = p.img + (size_t)nblk * kImg;
    p.cpl = p.inv + (size_t)nblk * kInvImg;
    p.slot = p.cpl + (size_t)nnode * kCplImg;
  }
  const bool m_is_a = p.left != p.trans;  // M is A itself, else A^T
  const int64_t mi = m_is_a ? 1 : p.lda, mk = m_is_a ? p.lda : 1;
  const int rev = p.forward ? 0 : 1;
  // diagonal blocks, then (node path) one block per 16-row strip of each
  // node's coupling block
  trsm_pack_kernel<<<dim3((unsigned)(nblk + (p.nodes ? nnode : 0)), kLeaf / 16), 256, 0, p.ctx->stream>>>(
      order, p.A, p.lda, mi, mk, rev, p.unit, p.img, p.slot, nblk, p.cpl);
  WGB_CHECK_LAUNCH("trsm_pack_kernel");
  if (p.nodes) {
    trsm_invert_kernel<<<dim3(kSub, (unsigned)nblk), 256, 0, p.ctx->stream>>>(order, p.img, p.inv, p.slot);
    WGB_CHECK_LAUNCH("trsm_invert_kernel");
  }
  return WGB_OK;
}

// Solves the node of frame rows [lo, hi) (lo a multiple of kNode, at most
// kNode rows: block P = [lo, lo + 256), block Q the rest) with the right-hand
// sides scaled by alpha as they are read. F, the block solved first, is P
// forward and Q backward.
int trsm_node(const Trsm &p, int64_t lo, int64_t hi, float alpha) {
  const int64_t nbP = hi - lo < kLeaf ? hi - lo : kLeaf, nbQ = hi - lo - nbP;
  const bool two = nbQ > 0;
  const int64_t sF = (!p.forward && two) ? lo + kLeaf : lo;
  const int64_t sS = p.forward ? lo + kLeaf : lo;
  auto at = [&](int64_t start) { return p.left ? p.B + start : p.B + start * p.ldb; };
  NodeArgs a;
  a.nbF = (int)(sF == lo ? nbP : nbQ);
  a.nbS = two ? (int)(sS == lo ? nbP : nbQ) : 0;
  a.rev = p.forward ? 0 : 1;
  a.nrhs = p.left ? p.n : p.m;
  a.vi = p.left ? 1 : p.ldb;
  a.vr = p.left ? p.ldb : 1;
  a.BF = at(sF);
  a.BS = two ? at(sS) : a.BF;
  a.alpha = alpha;
  const int64_t lF = sF / kLeaf, lS = two ? sS / kLeaf : lF;
  a.imgF = p.img + lF * kImg;
  a.imgS = p.img + lS * kImg;
  a.invF = p.inv + lF * kInvImg;
  a.invS = p.inv + lS * kInvImg;
  a.slotF = p.slot + lF * 32;
  a.slotS = p.slot + lS * 32;
  a.cpl = p.cpl + (lo / kNode) * kCplImg;
  trsm_node_kernel<<<(unsigned)((a.nrhs + 15) / 16), 256, 0, p.ctx->stream>>>(a);
  WGB_CHECK_LAUNCH("trsm_node_kernel");
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

// trsm_solve on the node path: nodes of kNode rows, the same halving and
// updates above them.
int trsm_solve_nodes(const Trsm &p, int64_t lo, int64_t hi, bool scaled) {
  const int64_t size = hi - lo;
  if (size <= kNode) return trsm_node(p, lo, hi, scaled ? 1.f : p.alpha);
  const int64_t mid = lo + (size / 2 + kNode - 1) / kNode * kNode;
  const int64_t a0 = p.forward ? lo : mid, a1 = p.forward ? mid : hi;
  const int64_t b0 = p.forward ? mid : lo, b1 = p.forward ? hi : mid;
  int st = trsm_solve_nodes(p, a0, a1, scaled);
  if (st) return st;
  if ((st = trsm_update(p, a0, a1 - a0, b0, b1 - b0, scaled ? 1.f : p.alpha))) return st;
  return trsm_solve_nodes(p, b0, b1, true);
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

namespace {

template <typename T>
int gemm_t(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t m, int64_t n, int64_t k,
           T alpha, const T *A, int64_t lda, const T *B, int64_t ldb, T beta, T *C, int64_t ldc,
           int band) {
  if constexpr (sizeof(T) == 4)
    return wgb::gemm_f32(ctx, uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                         band);
  else
    return wgb::gemm_f64(ctx, uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                         band);
}

// C = alpha op(A) op(B), one operand banded, its diagonal blocks from side.
template <typename T>
int gemm_side_t(wgb_ctx *ctx, int transA, int transB, int64_t m, int64_t n, int64_t k, T alpha,
                const T *A, int64_t lda, const T *B, int64_t ldb, T *C, int64_t ldc, int band,
                const T *side) {
  if constexpr (sizeof(T) == 4)
    return wgb::gemm_side_f32(ctx, transA, transB, m, n, k, alpha, A, lda, B, ldb, C, ldc, band, side);
  else
    return wgb::gemm_side_f64(ctx, transA, transB, m, n, k, alpha, A, lda, B, ldb, C, ldc, band, side);
}

// ssyr2k / dsyr2k. fp64 keeps reference BLAS's quick return
// (src/dsyr2k/dsyr2k.mjs:172-174): alpha = 0 or k = 0 with beta = 1 leaves C.
template <typename T>
int syr2k(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t n, int64_t k, T alpha,
          const T *A, int64_t lda, const T *B, int64_t ldb, T beta, T *C, int64_t ldc) {
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
  if (sizeof(T) == 8 && (alpha == (T)0 || k == 0) && beta == (T)1) return WGB_OK;
  wgb::timing_begin(ctx);
  if (transA == transB && lda == ldb) {
    // op(A) op(B)^T and op(B) op(A)^T take the same GEMM layout and leading
    // dimensions: one launch over k-tiles of (A, B) then of (B, A), both
    // products summed in one accumulator and alpha applied once. (wgblas
    // runs its GEMM twice, the second pass with beta = 1,
    // src/ssyr2k/ssyr2k.mjs:206-262: the same products, rounded once more.)
    if constexpr (sizeof(T) == 4)
      st = wgb::gemm2_f32(ctx, uplo, transA, tBt, n, n, k, alpha, A, B, lda, B, A, ldb, beta, C, ldc);
    else
      st = wgb::gemm2_f64(ctx, uplo, transA, tBt, n, n, k, alpha, A, B, lda, B, A, ldb, beta, C, ldc);
    if (st) return st;
    wgb::timing_end(ctx);
    return WGB_OK;
  }
  // pass 1: alpha op(A) op(B)^T + beta C; pass 2: alpha op(B) op(A)^T + C
  // (src/ssyr2k/ssyr2k.mjs:206-262), one timed span
  if ((st = gemm_t<T>(ctx, uplo, transA, tBt, n, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                      wgb::kBandNone)))
    return st;
  if (alpha != (T)0 && k != 0 &&
      (st = gemm_t<T>(ctx, uplo, transB, tAt, n, n, k, alpha, B, ldb, A, lda, (T)1, C, ldc,
                      wgb::kBandNone)))
    return st;
  wgb::timing_end(ctx);
  return WGB_OK;
}

// ssymm / dsymm. fp64 keeps reference BLAS's quick return
// (src/dsymm/dsymm.mjs:143-145): alpha = 0 with beta = 1 leaves C.
template <typename T>
int symm(wgb_ctx *ctx, int side, int uplo, int transB, int64_t m, int64_t n, T alpha, const T *A,
         int64_t lda, const T *B, int64_t ldb, T beta, T *C, int64_t ldc) {
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
  if (!C || (alpha != (T)0 && (!A || !B))) return fail(WGB_ERR_INVALID_VALUE, "A, B or C is null");
  if (sizeof(T) == 8 && alpha == (T)0 && beta == (T)1) return WGB_OK;
  wgb::timing_begin(ctx);
  if (alpha == (T)0) {
    // C <- beta C, reading neither A nor B
    st = gemm_t<T>(ctx, 0, WGB_NO_TRANS, WGB_NO_TRANS, m, n, 0, (T)0, nullptr, 1, nullptr, 1, beta,
                   C, ldc, wgb::kBandNone);
  } else {
    const int64_t ldw = round4(order);
    if ((st = wgb::ensure_op_workspace(ctx, (size_t)ldw * order * sizeof(T)))) return st;
    T *W = static_cast<T *>(ctx->op_ws);
    const int64_t tiles = (order + kTile - 1) / kTile;
    symmetrize_kernel<T><<<dim3((unsigned)tiles, (unsigned)tiles), 256, 0, ctx->stream>>>(
        order, A, lda, uplo, W, ldw);
    WGB_CHECK_LAUNCH("symmetrize_kernel");
    st = side == WGB_LEFT
             ? gemm_t<T>(ctx, 0, WGB_NO_TRANS, transB, m, n, m, alpha, W, ldw, B, ldb, beta, C, ldc,
                         wgb::kBandNone)
             : gemm_t<T>(ctx, 0, transB, WGB_NO_TRANS, m, n, n, alpha, B, ldb, W, ldw, beta, C, ldc,
                         wgb::kBandNone);
  }
  if (st) return st;
  wgb::timing_end(ctx);
  return WGB_OK;
}

// strmm / dtrmm: B copied, the triangle's diagonal blocks copied with zeros
// in the other triangle, one GEMM whose tiles run only the k-tiles the
// triangle reaches (banded tiles), reading the triangle in place outside its
// diagonal blocks (wgblas's dtrmm multiplies a whole dense copy,
// src/dtrmm/dtrmm.mjs:21-27).
template <typename T>
int trmm(wgb_ctx *ctx, int side, int uplo, int transA, int diag, int64_t m, int64_t n, T alpha,
         const T *A, int64_t lda, T *B, int64_t ldb) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_tri(side, uplo, transA, diag, m, n, A, lda, B, ldb))) return st;
  if (m == 0 || n == 0) return WGB_OK;
  wgb::timing_begin(ctx);
  if (alpha == (T)0) {
    // B <- 0, reading neither A nor B
    st = gemm_t<T>(ctx, 0, WGB_NO_TRANS, WGB_NO_TRANS, m, n, 0, (T)0, nullptr, 1, nullptr, 1, (T)0,
                   B, ldb, wgb::kBandNone);
  } else {
    const bool left = side == WGB_LEFT;
    const int64_t order = left ? m : n;
    // W: the triangle's diagonal blocks at A's leading dimension; Bc: B's
    // copy (the product overwrites B), 16-byte aligned after W
    const int64_t wlen = round4(lda * order), ldbc = round4(m);
    if ((st = wgb::ensure_op_workspace(ctx, (size_t)(wlen + ldbc * n) * sizeof(T)))) return st;
    T *W = static_cast<T *>(ctx->op_ws);
    T *Bc = W + wlen;
    const int64_t nblk = (order + wgb::kSideBlock - 1) / wgb::kSideBlock;
    diag_copy_kernel<T><<<dim3((unsigned)nblk, wgb::kSideBlock / 8), 256, 0, ctx->stream>>>(
        order, A, lda, uplo, diag == WGB_UNIT, W);
    WGB_CHECK_LAUNCH("diag_copy_kernel");
    WGB_CHECK_HIP(hipMemcpy2DAsync(Bc, (size_t)ldbc * sizeof(T), B, (size_t)ldb * sizeof(T),
                                   (size_t)m * sizeof(T), (size_t)n, hipMemcpyDeviceToDevice,
                                   ctx->stream));
    const bool op_lower = (uplo == WGB_LOWER) != (transA == WGB_TRANS);
    st = left ? gemm_side_t<T>(ctx, transA, WGB_NO_TRANS, m, n, m, alpha, A, lda, Bc, ldbc, B, ldb,
                               op_lower ? wgb::kBandALower : wgb::kBandAUpper, W)
              : gemm_side_t<T>(ctx, WGB_NO_TRANS, transA, m, n, n, alpha, Bc, ldbc, A, lda, B, ldb,
                               op_lower ? wgb::kBandBLower : wgb::kBandBUpper, W);
  }
  if (st) return st;
  wgb::timing_end(ctx);
  return WGB_OK;
}

}  // namespace

extern "C" int wgb_ssyr2k(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t n, int64_t k,
                          float alpha, const float *A, int64_t lda, const float *B, int64_t ldb,
                          float beta, float *C, int64_t ldc) {
  return syr2k<float>(ctx, uplo, transA, transB, n, k, alpha, A, lda, B, ldb, beta, C, ldc);
}

extern "C" int wgb_dsyr2k(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t n, int64_t k,
                          double alpha, const double *A, int64_t lda, const double *B, int64_t ldb,
                          double beta, double *C, int64_t ldc) {
  return syr2k<double>(ctx, uplo, transA, transB, n, k, alpha, A, lda, B, ldb, beta, C, ldc);
}

extern "C" int wgb_ssymm(wgb_ctx *ctx, int side, int uplo, int transB, int64_t m, int64_t n,
                         float alpha, const float *A, int64_t lda, const float *B, int64_t ldb,
                         float beta, float *C, int64_t ldc) {
  return symm<float>(ctx, side, uplo, transB, m, n, alpha, A, lda, B, ldb, beta, C, ldc);
}

extern "C" int wgb_dsymm(wgb_ctx *ctx, int side, int uplo, int transB, int64_t m, int64_t n,
                         double alpha, const double *A, int64_t lda, const double *B, int64_t ldb,
                         double beta, double *C, int64_t ldc) {
  return symm<double>(ctx, side, uplo, transB, m, n, alpha, A, lda, B, ldb, beta, C, ldc);
}

extern "C" int wgb_strmm(wgb_ctx *ctx, int side, int uplo, int transA, int diag, int64_t m,
                         int64_t n, float alpha, const float *A, int64_t lda, float *B,
                         int64_t ldb) {
  return trmm<float>(ctx, side, uplo, transA, diag, m, n, alpha, A, lda, B, ldb);
}

extern "C" int wgb_dtrmm(wgb_ctx *ctx, int side, int uplo, int transA, int diag, int64_t m,
                         int64_t n, double alpha, const double *A, int64_t lda, double *B,
                         int64_t ldb) {
  return trmm<double>(ctx, side, uplo, transA, diag, m, n, alpha, A, lda, B, ldb);
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
    if (!(st = trsm_pack(p)))
      st = p.nodes ? trsm_solve_nodes(p, 0, p.left ? m : n, false) : trsm_solve(p, 0, p.left ? m : n, false);
  }
  if (st) return st;
  wgb::timing_end(ctx);
  return WGB_OK;
}
