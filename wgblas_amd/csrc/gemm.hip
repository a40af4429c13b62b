// GEMM family on CDNA4 matrix cores: sgemm, sgemmtr, ssyrk (fp32) and dgemm
// (native fp64).
//
// wgblas computes these with LDS-tiled, register-blocked WGSL kernels in a
// row-major frame (src/shaders/sgemm_large.wgsl, sgemm_small.wgsl) and
// emulates f64 with double-double pairs (src/shaders/dgemm_small.wgsl,
// src/shaders/f64/). Here the frame is column-major (BLAS's own) and the
// contraction runs on MFMA: v_mfma_f32_16x16x4f32 for fp32 and
// v_mfma_f64_16x16x4f64 for fp64, one template for both.
//
// Block: 256 threads = 4 waves in a 2x2 grid, block tile BT x BT of C
// (BT = 128 large tier, 64 small tier), k-tile BK = 128 bytes of k (32
// floats / 16 doubles); tiny fp32 problems take a
// one-launch kernel of 32x32 tiles (gemm_small_kernel), and large fp32
// problems of whole 256 x 128 tiles the wide tier (gemm_wide_kernel: 16-float
// k-tiles, 128 x 64 wave tiles, two blocks per CU). Each operand tile is
// staged in LDS, double buffered, in the orientation it has in memory so the
// global->LDS path is plain 16-byte copies (for 16-byte aligned operands,
// copies made by global_load_lds_dwordx4 without passing through
// registers):
//   * k-contiguous operands (op(A) with A transposed, op(B) with B not
//     transposed) are stored [row][k], 128-byte rows whose eight 16-byte
//     chunks are XOR-swizzled by row (kc_swz) so that both the stores and
//     the 16-row operand reads touch every LDS bank once;
//   * mn-contiguous operands (A not transposed, B transposed) are stored
//     [k][row].
// MFMA operand fetch from either layout is one 16-byte (or 8-byte) LDS read
// per lane:
//   * from [row][k], a lane reads 4 consecutive k and feeds them to 4
//     successive MFMAs: in MFMA step s lane-group g = lane/16 supplies
//     k = 4g + s (the k order inside a 16-k chunk is permuted the same way
//     for both operands, so the sum is unchanged);
//   * from [k][row], a lane reads RW consecutive rows and feeds each to a
//     different 16-row MFMA block ("virtual blocks"), which permutes rows
//     inside the wave tile; the epilogue undoes it.
// Each lane therefore holds runs of consecutive C rows, which the epilogue
// writes as 16-byte vectors when alignment allows.
//
// Tiles are scheduled XCD-aware: the hardware deals workgroups round-robin
// over MI355X's 8 XCDs, so workgroup w is remapped to logical tile
// (w % 8) * (tiles / 8) + w / 8, giving each XCD (and its L2) a contiguous
// run of tiles; inside that run tiles are grouped 8 tile-rows at a time so
// concurrent tiles share A and B panels. sgemmtr/ssyrk launch only the
// tiles that meet the requested triangle (wgblas launches all of them and
// returns early, src/shaders/sgemm_large.wgsl:78-83), in bands of 4 tile rows
// walked column by column for the same sharing, and mask stores inside the
// diagonal tiles (tile_order.h holds these orders).
//
// Result rules kept from wgblas (src/shaders/sgemm_large.wgsl:288-308,
// src/shaders/dgemm_small.wgsl:230-273): beta == 0 never reads C;
// alpha == 0 (and k == 0) gives beta*C without reading A or B; rows and
// columns outside m x n, and the other triangle for sgemmtr/ssyrk, are
// never written.
#include "common.h"
#include "tile_order.h"

#include <cmath>
#include <string>
#include <type_traits>

namespace {

template <typename T>
struct Ty;

template <>
struct Ty<float> {
  typedef float v16 __attribute__((ext_vector_type(4)));
  typedef float v4 __attribute__((ext_vector_type(4)));
  typedef float v2 __attribute__((ext_vector_type(2)));
  typedef float acc __attribute__((ext_vector_type(4)));
  static constexpr int VW = 4;
  // Row of the 16x16 result held by accumulator register q of lane-group g
  // (lane / 16): rows 4g .. 4g+3 (checked on gfx950 with one-hot operands).
  __device__ static int drow(int g, int q) { return 4 * g + q; }
  __device__ static acc mfma(float a, float b, acc c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

template <>
struct Ty<double> {
  typedef double v16 __attribute__((ext_vector_type(2)));
  typedef double v4 __attribute__((ext_vector_type(4)));
  typedef double v2 __attribute__((ext_vector_type(2)));
  typedef double acc __attribute__((ext_vector_type(4)));
  static constexpr int VW = 2;
  // The fp64 16x16x4 MFMA interleaves instead: register q of lane-group g
  // holds row g + 4q.
  __device__ static int drow(int g, int q) { return g + 4 * q; }
  __device__ static acc mfma(double a, double b, acc c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
  }
};

template <typename T>
struct GemmArgs {
  int64_t m, n, k;
  T alpha, beta;
  const T *A;
  int64_t lda;
  const T *B;
  int64_t ldb;
  T *C;
  int64_t ldc;
  int tiles_m, tiles_n, ntiles;
  int uplo;   // 0 = full C, WGB_LOWER, WGB_UPPER
  int c_vec;  // interior tiles store C in vectors (fp32 always; fp64 if C is 16-byte aligned)
  // wgb::kBand*: one operand is triangular (zero outside its triangle), so a
  // tile only needs the k-tiles its nonzero band reaches (never split).
  int band;
  // Split-k tail: logical tiles [nregular, ntiles) are computed as `splits`
  // k-ranges of kt_split k-tiles each; unit u = (tile - nregular) * splits +
  // split writes its raw BT x BT partial (column-major, ld BT) to ws + u BT^2
  // and split_fixup adds them. nregular == ntiles: no split.
  int nregular, splits, kt_split;
  T *ws;
  // Two-part k range (K2 kernels, ssyr2k / dsyr2k as one launch): k-tiles
  // kt >= kt_switch read A2 in place of A and B2 in place of B, at the same
  // leading dimensions and at k-tile kt - kt_switch of those.
  const T *A2, *B2;
  int kt_switch;
  // Banded GEMMs (paired kernels): with band_side set, the banded operand's
  // diagonal kSideBlock x kSideBlock blocks are read from A2 (band on A) or
  // B2 (band on B) at the same leading dimension and element coordinates,
  // everything else from A / B in place (trmm: the caller's triangle stays
  // where it is; only its diagonal blocks are copied, the other triangle
  // zeroed in them).
  int band_side;
};

constexpr int kThreads = 256;

// global_load_lds_dwordx4: each lane copies 16 bytes from its own global
// address to LDS at `lds` (wave-uniform, set in M0) + 16 * lane.
__device__ __forceinline__ void copy16_to_lds(const void *g, void *lds) {
  typedef __attribute__((address_space(3))) void *LdsPtr;
  __builtin_amdgcn_global_load_lds(g, (LdsPtr)lds, 16, 0, 0);
}
// Instruction classes of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedVmemRead = 0x020;
constexpr int kSchedDsRead = 0x100;
constexpr int kSchedDsWrite = 0x200;
using wgb_tiles::logical_tile;
using wgb_tiles::triangle_tiles;
using wgb_tiles::xcd_remap;

// Chunk position of 16-byte chunk c of staged row r in the [row][k] layout
// is c ^ kc_swz(r). A ds_write_b128 phase (8 lanes) fills one 128-byte row;
// a ds_read_b128 phase (16 lanes) reads one chunk of 16 consecutive rows.
// Measured on MI355X (SQ_LDS_BANK_CONFLICT, one wave per block, every
// 16-lane phase of the read pattern): the key r & 7 keeps both conflict-free,
// while a 16-byte row pad, or a key that also folds in row bit 3, costs a
// second cycle on every read.
__device__ __forceinline__ int kc_swz(int row) { return row & 7; }

// Global -> register -> LDS staging of one operand's BT x BK tile.
// KC: k-contiguous in memory, staged [row][k] (row stride BK, chunks
//     swizzled by kc_swz).
// !KC: row-contiguous in memory, staged [k][row] (row stride BT).
template <typename T, int BT, bool KC, bool VEC, int NT = kThreads, bool K2 = false>
struct Stager {
  typedef typename Ty<T>::v16 V;
  static constexpr int VW = Ty<T>::VW;
  static constexpr int BK = 128 / (int)sizeof(T);
  static constexpr int LOADS = BT * 8 / NT;  // 16-byte vectors per thread (NT threads)
  static constexpr int VPK = BT / VW;        // vectors per k-row (!KC)
  static constexpr int KROWS = NT / VPK;     // k-rows per load step (!KC)
  static constexpr int RPS = NT / 8;         // rows per load step (KC: 8 chunks per row)
  static constexpr int LDK = BK;
  static constexpr int LDM = BT;
  static constexpr int ELEMS = KC ? BT * LDK : BK * LDM;

  const T *base;      // this thread's element for k-tile 0, r = 0
  int64_t r_step;     // element distance between load steps r
  int64_t k_step;     // element advance per k-tile
  int lds_off;        // LDS element offset for r = 0
  int lds_r_step;
  int64_t row_first;  // KC: global row of r = 0;   !KC: first global row of the vector
  int k_first;        // KC: k offset of the vector; !KC: k-row of r = 0
  int64_t rows_total, K;
  // Edge tiles (set by init_edge), on whole k-tiles that are not the last
  // one: a lane whose rows are past rows_total (KC: load steps r >= nvr;
  // MC: vok false) reads at fb instead, row rows_total-1 of the same k. An
  // MC vector that is only partly in range reads up to VW-1 elements past
  // the end of its column; at least BK more columns of the matrix follow
  // (the last whole k-tile is not read this way), so the read stays inside
  // it for any ld. Values read for rows past rows_total only reach C rows /
  // columns that are never written, so they need not be zero, only be read
  // from inside the matrix.
  const T *fb;
  int nvr;
  bool vok;
  // LDS copies (load_lds): the wave-uniform origin of the operand tile at
  // k-tile 0 and this lane's byte offsets from it, one per load step.
  const T *origin;
  uint32_t voff[LOADS];
  int copy_shift;  // elements from this thread's register-path vector to its copy source
  // K2 (switchable stager): from k-tile ksw on, every address moves by dsw
  // bytes. Two-part k: k-tile kt of the first operand's addressing becomes
  // k-tile kt - kt_switch of the second operand (same leading dimension, so
  // the same offsets from it). Side copy: the same element coordinates in
  // the second matrix (same leading dimension).
  int ksw;
  int64_t dsw;

  // After init (k_step set), before advance.
  __device__ void set_switch(const T *P, const T *P2, int kt_switch) {
    ksw = kt_switch;
    dsw = ((const char *)P2 - (const char *)P) - (int64_t)kt_switch * k_step * (int64_t)sizeof(T);
  }
  // Side copy: k-tiles from kt_sw on read P2's elements at P's coordinates.
  __device__ void set_side(const T *P, const T *P2, int kt_sw) {
    ksw = kt_sw;
    dsw = (const char *)P2 - (const char *)P;
  }
  __device__ const T *sel(const T *q, int kt) const {
    if constexpr (K2) return kt < ksw ? q : (const T *)((const char *)q + dsw);
    return q;
  }

  __device__ void init(const T *P, int64_t ld, int64_t row0, int t, int64_t rows_total_,
                       int64_t K_) {
    rows_total = rows_total_;
    K = K_;
    origin = KC ? P + row0 * ld : P + row0;
    if (KC) {
      int row = t / 8, kv = t % 8;
      row_first = row0 + row;
      k_first = kv * VW;
      base = P + (row0 + row) * ld + kv * VW;
      r_step = RPS * ld;
      k_step = BK;
      lds_off = row * LDK + (kv ^ kc_swz(row)) * VW;  // kc_swz(row + RPS r) == kc_swz(row)
      lds_r_step = RPS * LDK;
      // An LDS copy puts lane t at chunk t % 8 of the row, so that lane
      // reads the chunk the swizzle places there instead.
      copy_shift = ((kv ^ kc_swz(row)) - kv) * VW;
    } else {
      int mv = t % VPK, kk = t / VPK;
      row_first = row0 + mv * VW;
      k_first = kk;
      base = P + row0 + mv * VW + (int64_t)kk * ld;
      r_step = KROWS * ld;
      k_step = (int64_t)BK * ld;
      lds_off = kk * LDM + mv * VW;
      lds_r_step = KROWS * LDM;
      copy_shift = 0;
    }
  }

  // Moves the tile origin to k-tile kt0 (split-k ranges).
  __device__ void advance(int kt0) {
    base += (int64_t)kt0 * k_step;
    origin += (int64_t)kt0 * k_step;
    K -= (int64_t)kt0 * BK;
    if constexpr (K2) ksw -= kt0;
  }

  // Edge-tile fields (after init and advance): see the members above.
  __device__ void init_edge() {
    const int64_t valid = rows_total - row_first;  // rows of this thread in range (may be <= 0)
    if (KC) {
      const int64_t n = valid <= 0 ? 0 : (valid + RPS - 1) / RPS;
      nvr = (int)(n < LOADS ? n : LOADS);
      fb = base + (rows_total - 1 - row_first) * (r_step / RPS);
    } else {
      vok = valid > 0;
      fb = base + (rows_total - 1 - row_first);
    }
  }

  __device__ static V load_n(const T *p, int64_t nvalid) {
    V v;
#pragma unroll
    for (int c = 0; c < VW; ++c) v[c] = (c < nvalid) ? p[c] : (T)0;
    return v;
  }

  // One 16-byte load for any element-aligned p: CDNA multi-dword global
  // loads need dword alignment only. Typed with the element's alignment,
  // since the VEC path also takes fp32 operands that are not 16-byte
  // aligned.
  __device__ static V load_full(const T *p) {
    typedef T VU __attribute__((ext_vector_type(VW), aligned(sizeof(T))));
    return *reinterpret_cast<const VU *>(p);
  }

  // GUARD: k-tile past the end of K (element guards on rows and k);
  // otherwise a whole k-tile, with EDGE for tiles that cross rows_total.
  template <bool GUARD, bool EDGE = false>
  __device__ void load(V (&regs)[LOADS], int kt) const {
    const T *p = sel(base + (int64_t)kt * k_step, kt);
#pragma unroll
    for (int r = 0; r < LOADS; ++r) {
      const T *q = p + r * r_step;
      if (!GUARD && !EDGE) {
        regs[r] = load_full(q);
      } else if (!GUARD && KC) {
        regs[r] = load_full(r < nvr ? q : sel(fb + (int64_t)kt * k_step, kt));
      } else if (!GUARD) {
        regs[r] = load_full(vok ? q : sel(fb + (int64_t)kt * k_step, kt) + r * r_step);
      } else if (KC) {
        int64_t row = row_first + 32 * r;
        int64_t nv = K - ((int64_t)kt * BK + k_first);
        regs[r] = (row < rows_total && nv > 0) ? (nv >= VW ? load_full(q) : load_n(q, nv)) : V(0);
      } else {
        int64_t kk = (int64_t)kt * BK + k_first + KROWS * r;
        int64_t nv = rows_total - row_first;
        regs[r] = (kk < K && nv > 0) ? (nv >= VW ? load_full(q) : load_n(q, nv)) : V(0);
      }
    }
  }

  // Lane offsets for load_lds, after init, advance and (EDGE) init_edge.
  // They fit in 32 bits: the host sends operands with BT * ld * sizeof(T)
  // of 2^31 or more down the register path (VEC false).
  template <bool EDGE>
  __device__ void init_copy() {
#pragma unroll
    for (int r = 0; r < LOADS; ++r) {
      const T *q = base + r * r_step;
      if (EDGE && KC) q = r < nvr ? q : fb;
      if (EDGE && !KC) q = vok ? q : fb + r * r_step;
      voff[r] = (uint32_t)((const char *)(q + copy_shift) - (const char *)origin);
    }
  }

  // Whole k-tile kt copied straight from global memory into `stage` with
  // global_load_lds_dwordx4 (no registers): lane l of wave w lands at
  // 16 l bytes past a wave-uniform address, i.e. thread t's vector r at
  // element VW t + r lds_r_step. In the [k][row] layout that is where store()
  // puts it; in the [row][k] layout it is chunk t % 8 of row t / 8, so the
  // lane reads the global chunk the swizzle maps there (copy_shift), and the
  // stage ends up exactly as store() would leave it. Completion is tracked
  // by vmcnt; readers wait for it and then a barrier.
  // SCALAR_BASE: the address is the scalar tile origin plus a 32-bit lane
  // offset (the instruction's saddr + voffset form); the empty asm
  // statements keep the compiler from strength-reducing it into per-lane
  // 64-bit pointers. Otherwise it does exactly that (two VALU operations
  // and two VGPRs per copy). Which is faster depends on the kernel.
  template <bool EDGE, bool SCALAR_BASE>
  __device__ void load_lds(T *stage, int kt, int wave) const {
    static_assert(sizeof(V) == 16, "LDS copies move 16 bytes per lane");
    T *dst = stage + wave * 64 * VW;
    if constexpr (SCALAR_BASE) {
      const uint64_t o64 = (uint64_t)sel(origin + (int64_t)kt * k_step, kt);
      uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)o64);
      uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(o64 >> 32));
      asm volatile("" : "+s"(lo), "+s"(hi));
      const char *o = (const char *)(((uint64_t)hi << 32) | lo);
#pragma unroll
      for (int r = 0; r < LOADS; ++r) {
        uint32_t v = voff[r];
        asm volatile("" : "+v"(v));
        copy16_to_lds(o + v, dst + r * lds_r_step);
      }
    } else {
      const T *p = sel(base + (int64_t)kt * k_step, kt);
#pragma unroll
      for (int r = 0; r < LOADS; ++r) {
        const T *q = p + r * r_step;
        if (EDGE && KC) q = r < nvr ? q : sel(fb + (int64_t)kt * k_step, kt);
        if (EDGE && !KC) q = vok ? q : sel(fb + (int64_t)kt * k_step, kt) + r * r_step;
        copy16_to_lds(q + copy_shift, dst + r * lds_r_step);
      }
    }
  }

  __device__ void store(T *stage, const V (&regs)[LOADS]) const {
#pragma unroll
    for (int r = 0; r < LOADS; ++r)
      *reinterpret_cast<V *>(stage + lds_off + r * lds_r_step) = regs[r];
  }
};

// Fetches the MFMA operands of one 16-k chunk for MB 16-row blocks.
// out[s][b] = operand of MFMA step s (s = 0..3) for block b.
template <typename T, int BT, bool KC, int MB>
__device__ __forceinline__ void fetch_operands(const T *stage, int wrow, int kc, int lane,
                                               T (&out)[4][MB]) {
  typedef typename Ty<T>::v4 V4;
  constexpr int VW = Ty<T>::VW;
  constexpr int BK = 128 / (int)sizeof(T);
  constexpr int LDK = BK;
  constexpr int LDM = BT;
  constexpr int RW = MB < VW ? MB : VW;
  const int g = lane >> 4, i16 = lane & 15;
  if (KC) {
    // wrow is a multiple of 16, so the row key is kc_swz(i16); the 4 k of
    // lane group g are 4 / VW whole chunks.
    const int key = kc_swz(i16);
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      const T *row = stage + (wrow + 16 * b + i16) * LDK;
      if (VW == 4) {
        V4 v = *reinterpret_cast<const V4 *>(row + ((((kc + 4 * g) / VW) ^ key) * VW));
#pragma unroll
        for (int s = 0; s < 4; ++s) out[s][b] = v[s];
      } else {
        typedef typename Ty<T>::v2 V2;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          V2 v = *reinterpret_cast<const V2 *>(row + ((((kc + 4 * g) / VW + h) ^ key) * VW));
          out[2 * h][b] = v[0];
          out[2 * h + 1][b] = v[1];
        }
      }
    }
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int h = 0; h < MB / RW; ++h) {
        const T *p = stage + (kc + 4 * g + s) * LDM + wrow + 16 * RW * h + RW * i16;
        if (RW == 4) {
          V4 v = *reinterpret_cast<const V4 *>(p);
#pragma unroll
          for (int c = 0; c < RW; ++c) out[s][h * RW + c] = v[c];
        } else {
          typedef typename Ty<T>::v2 V2;
          V2 v = *reinterpret_cast<const V2 *>(p);
#pragma unroll
          for (int c = 0; c < RW; ++c) out[s][h * RW + c] = v[c];
        }
      }
    }
  }
}

// Fetches the MFMA operands of step s of one 16-k chunk for MB 16-row
// blocks: out[b] = operand of block b. Same data as fetch_operands, issued
// step by step so only one step's operands are live (used where register
// pressure, not LDS instruction count, limits occupancy).
template <typename T, int BT, bool KC, int MB>
__device__ __forceinline__ void fetch_step(const T *stage, int wrow, int kc, int s, int lane,
                                           T (&out)[MB]) {
  constexpr int VW = Ty<T>::VW;
  constexpr int BK = 128 / (int)sizeof(T);
  constexpr int LDK = BK;
  constexpr int LDM = BT;
  constexpr int RW = MB < VW ? MB : VW;
  const int g = lane >> 4, i16 = lane & 15;
  if (KC) {
    const int kk = kc + 4 * g + s;
    const int off = (((kk / VW) ^ kc_swz(i16)) * VW) + kk % VW;
#pragma unroll
    for (int b = 0; b < MB; ++b) out[b] = stage[(wrow + 16 * b + i16) * LDK + off];
  } else {
#pragma unroll
    for (int h = 0; h < MB / RW; ++h) {
      const T *p = stage + (kc + 4 * g + s) * LDM + wrow + 16 * RW * h + RW * i16;
      if (RW == 4) {
        typedef typename Ty<T>::v4 V4;
        V4 v = *reinterpret_cast<const V4 *>(p);
#pragma unroll
        for (int c = 0; c < RW; ++c) out[h * RW + c] = v[c];
      } else {
        typedef typename Ty<T>::v2 V2;
        V2 v = *reinterpret_cast<const V2 *>(p);
#pragma unroll
        for (int c = 0; c < RW; ++c) out[h * RW + c] = v[c];
      }
    }
  }
}

// Row inside the wave tile held by lane `lane` for MFMA block b and
// accumulator register q.
template <typename T, bool KC, int MB>
__device__ __forceinline__ int out_row(int b, int q, int lane) {
  constexpr int VW = Ty<T>::VW;
  constexpr int RW = MB < VW ? MB : VW;
  const int r = Ty<T>::drow(lane >> 4, q);
  if (KC) return 16 * b + r;
  return 16 * RW * (b / RW) + RW * r + (b % RW);
}

// Column inside the wave tile held by lane `lane` for MFMA block b.
template <bool KC, int MB, int VW>
__device__ __forceinline__ int out_col(int b, int lane) {
  constexpr int RW = MB < VW ? MB : VW;
  const int i16 = lane & 15;
  if (KC) return 16 * b + i16;
  return 16 * RW * (b / RW) + RW * i16 + (b % RW);
}

// Epilogue of a whole interior tile with C accessed in vectors (fp32: any
// C; fp64: ldc a multiple of the vector width, C 16-byte aligned; vector
// types of element alignment). Every lane holds runs of
// consecutive C rows in one column:
//   * A mn-contiguous: blocks i = RW h + c (c = 0..RW-1) of register q sit at
//     rows 16 RW h + RW drow(g, q) + c, a run of RW rows;
//   * A k-contiguous, fp32: registers q = 0..3 of block i sit at rows
//     16 i + 4 g + q, a run of 4 rows.
// (fp64 with A k-contiguous holds no runs: drow interleaves; it keeps the
// scalar path.) All C loads of a batch are issued before any store.
template <typename T, bool AKC, bool BKC, int MA, int MN, bool ONE_COL = false>
__device__ __forceinline__ void epilogue_vec(const GemmArgs<T> &p,
                                             const typename Ty<T>::acc (&acc)[MA][MN],
                                             int64_t row0, int64_t col0, int lane) {
  constexpr int VW = Ty<T>::VW;
  constexpr int RW = MA < VW ? MA : VW;
  const int g = lane >> 4;
  const T alpha = p.alpha, beta = p.beta;
  if constexpr (!AKC) {
    // element alignment: fp32 C may start anywhere dword-aligned
    typedef T VN __attribute__((ext_vector_type(RW), aligned(sizeof(T))));
    // fp32 keeps every column block in flight at once; fp64 (accumulators
    // in VGPRs) and ONE_COL go one column block at a time.
    constexpr int JB = (sizeof(T) == 4 && !ONE_COL) ? MN : 1;
#pragma unroll
    for (int j0 = 0; j0 < MN; j0 += JB) {
      VN cv[JB][MA / RW][4];
      T *cp[JB][MA / RW][4];
#pragma unroll
      for (int jj = 0; jj < JB; ++jj) {
        const int64_t col = col0 + out_col<BKC, MN, VW>(j0 + jj, lane);
#pragma unroll
        for (int h = 0; h < MA / RW; ++h)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            cp[jj][h][q] = p.C + (row0 + 16 * RW * h + RW * Ty<T>::drow(g, q)) + col * p.ldc;
            if (beta != (T)0) cv[jj][h][q] = *reinterpret_cast<const VN *>(cp[jj][h][q]);
          }
      }
#pragma unroll
      for (int jj = 0; jj < JB; ++jj)
#pragma unroll
        for (int h = 0; h < MA / RW; ++h)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            VN v;
#pragma unroll
            for (int c = 0; c < RW; ++c) {
              T x = alpha * acc[h * RW + c][j0 + jj][q];
              v[c] = beta != (T)0 ? fma(beta, cv[jj][h][q][c], x) : x;
            }
            *reinterpret_cast<VN *>(cp[jj][h][q]) = v;
          }
    }
  } else {
    static_assert(sizeof(T) == 4, "vector epilogue with k-contiguous A is fp32 only");
    typedef T V4 __attribute__((ext_vector_type(4), aligned(sizeof(T))));
    if constexpr (ONE_COL) {
#pragma unroll
      for (int j = 0; j < MN; ++j) {
        const int64_t col = col0 + out_col<BKC, MN, VW>(j, lane);
        V4 cv[MA];
        T *cp[MA];
#pragma unroll
        for (int i = 0; i < MA; ++i) {
          cp[i] = p.C + (row0 + 16 * i + 4 * g) + col * p.ldc;
          if (beta != (T)0) cv[i] = *reinterpret_cast<const V4 *>(cp[i]);
        }
#pragma unroll
        for (int i = 0; i < MA; ++i) {
          V4 v;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            T x = alpha * acc[i][j][q];
            v[q] = beta != (T)0 ? fma(beta, cv[i][q], x) : x;
          }
          *reinterpret_cast<V4 *>(cp[i]) = v;
        }
      }
      return;
    }
    V4 cv[MA][MN];
    T *cp[MA][MN];
#pragma unroll
    for (int i = 0; i < MA; ++i)
#pragma unroll
      for (int j = 0; j < MN; ++j) {
        const int64_t col = col0 + out_col<BKC, MN, VW>(j, lane);
        cp[i][j] = p.C + (row0 + 16 * i + 4 * g) + col * p.ldc;
        if (beta != (T)0) cv[i][j] = *reinterpret_cast<const V4 *>(cp[i][j]);
      }
#pragma unroll
    for (int i = 0; i < MA; ++i)
#pragma unroll
      for (int j = 0; j < MN; ++j) {
        V4 v;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          T x = alpha * acc[i][j][q];
          v[q] = beta != (T)0 ? fma(beta, cv[i][j][q], x) : x;
        }
        *reinterpret_cast<V4 *>(cp[i][j]) = v;
      }
  }
}

// fp64 fetches operands per MFMA step and is held to two waves per SIMD
// (256 registers): its 128 accumulator registers leave no room for a whole
// chunk of operands at that occupancy. fp32 fetches a chunk at a time.
template <typename T>
struct KernelPolicy {
  static constexpr bool kPerStep = sizeof(T) == 8;
};

// Waits until this wave's global -> LDS copies (vmcnt) and LDS operations
// (lgkmcnt) are complete, then joins the block barrier: after it, every
// wave's copies are visible in LDS.
__device__ __forceinline__ void copies_landed_sync() {
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) expcnt(7) lgkmcnt(0)
  __syncthreads();
}

// One BTM x BTN tile (tm, tn) of C over k-tiles [kt0, kt0 + nkt): the main
// loop and the epilogue (unit >= 0: a split-k unit's raw partial to ws).
// NT = 256 threads (2 x 2 waves); every wave owns a square WT x WT part of
// the tile.
template <typename T, int BTM, int BTN, int NT, bool AKC, bool BKC, bool VEC, bool K2 = false,
          bool SIDE = false>
__device__ __forceinline__ void gemm_tile(const GemmArgs<T> &p, int tm, int tn, int unit, int kt0,
                                          int nkt, T *smem, const int t) {
  typedef typename Ty<T>::acc Acc;
  typedef typename Ty<T>::v16 V;
  constexpr int VW = Ty<T>::VW;
  constexpr int BK = 128 / (int)sizeof(T);
  static_assert(NT == 256, "2 x 2 waves per block");
  constexpr int WGM = 2;  // waves along m
  constexpr int WT = BTM / WGM;
  static_assert(WT == BTN / (NT / 64 / WGM), "square wave tiles");
  constexpr int MB = WT / 16;
  typedef Stager<T, BTM, AKC, VEC, NT, K2 || SIDE> SA;
  typedef Stager<T, BTN, BKC, VEC, NT, K2 || SIDE> SB;
  constexpr int STAGE = SA::ELEMS + SB::ELEMS;
  const int64_t m0 = (int64_t)tm * BTM, n0 = (int64_t)tn * BTN;
  const int lane = t & 63, wave = t >> 6;
  const int wm = (wave % WGM) * WT, wn = (wave / WGM) * WT;

  // k-tiles are counted from kt0 below: the stagers start at k = kt0 BK and
  // see K - kt0 BK columns.
  SA sa;
  SB sb;
  if constexpr (SIDE) {
    // Banded operand with a side copy of its diagonal blocks: the k-tiles of
    // this tile's diagonal block come from the copy, the rest in place. A
    // band that starts at the diagonal (op(A) upper, op(B) lower) reads the
    // copy first; one that ends there (op(A) lower, op(B) upper) reads it
    // last. Without a side copy no k-tile switches.
    constexpr int kSideTiles = wgb::kSideBlock / BK;  // k-tiles per diagonal block
    const T *PA = p.A, *QA = p.A, *PB = p.B, *QB = p.B;
    int kswA = INT32_MAX, kswB = INT32_MAX;
    if (p.band_side) {
      const int da = (int)(m0 / wgb::kSideBlock), db = (int)(n0 / wgb::kSideBlock);
      if (p.band == wgb::kBandALower) {
        QA = p.A2;
        kswA = da * kSideTiles;
      } else if (p.band == wgb::kBandAUpper) {
        PA = p.A2;
        kswA = (da + 1) * kSideTiles;
      } else if (p.band == wgb::kBandBLower) {
        PB = p.B2;
        kswB = (db + 1) * kSideTiles;
      } else if (p.band == wgb::kBandBUpper) {
        QB = p.B2;
        kswB = db * kSideTiles;
      }
    }
    sa.init(PA, p.lda, m0, t, p.m, p.k);
    sb.init(PB, p.ldb, n0, t, p.n, p.k);
    sa.set_side(PA, QA, kswA);
    sb.set_side(PB, QB, kswB);
  } else {
    sa.init(p.A, p.lda, m0, t, p.m, p.k);
    sb.init(p.B, p.ldb, n0, t, p.n, p.k);
  }
  if constexpr (K2) {
    sa.set_switch(p.A, p.A2, p.kt_switch);
    sb.set_switch(p.B, p.B2, p.kt_switch);
  }
  sa.advance(kt0);
  sb.advance(kt0);
  const bool interior = (m0 + BTM <= p.m) && (n0 + BTN <= p.n);
  const int nkt_full = (int)(p.k / BK) - kt0;  // whole k-tiles from kt0

  Acc acc[MB][MB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[i][j] = Acc(0);

  // Main loop, instantiated once for interior tiles and once for edge tiles
  // (rows past m or columns past n: whole k-tiles take the EDGE loads).
  auto mainloop = [&](auto edge_tag) {
    constexpr bool EDGE = decltype(edge_tag)::value;
    if constexpr (EDGE) {
      sa.init_edge();
      sb.init_edge();
    }
    // Whole k-tiles taking unguarded (or EDGE) loads; an edge tile's last
    // whole k-tile is guarded too (EDGE reads may run past a column end).
    const int nkt_whole = EDGE ? nkt_full - 1 : nkt_full;
    if constexpr (sizeof(T) == 4 && VEC) {
      // fp32 with 16-byte aligned operands: whole k-tiles are copied from
      // global memory straight into LDS (load_lds); a partial last k-tile
      // (and an edge tile's last whole one) takes the guarded register path.
      // Two LDS buffers, two 16-k chunks per k-tile. On entry to iteration
      // kt: X = chunk 0 of tile kt (registers), tile kt in buffer kt&1, the
      // copies of tile kt+1 into buffer (kt+1)&1 issued.
      //   1. LDS reads of chunk 1 of tile kt into Y
      //   2. MFMAs on X
      //   3. wait for this wave's copies, barrier: tile kt+1 is complete in
      //      buffer (kt+1)&1, and every wave is done reading buffer kt&1
      //   4. copies of tile kt+2 into buffer kt&1
      //   5. LDS reads of chunk 0 of tile kt+1 into X
      //   6. MFMAs on Y
      // A copy has a whole k-tile of MFMAs (steps 6, 1, 2) to land, and no
      // registers or LDS store instructions are spent on staging.
      static_assert(BK == 32, "the pipelined fp32 loop assumes two 16-k chunks per k-tile");
      // Scalar-base copies (scalar tile origin + 32-bit lane offsets):
      // measured against per-lane 64-bit pointers at 8192^3 on one box, NT
      // 144.6 -> 147.1 TFLOP/s and ssyrk 8192/4096 138.9 -> 141.1, the other
      // layouts (which already used them) unchanged.
      constexpr bool kScalarBase = true;
      const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
      sa.template init_copy<EDGE>();
      sb.template init_copy<EDGE>();
      auto fill = [&](int kt) {
        T *st = smem + (kt & 1) * STAGE;
        if (kt < nkt_whole) {
          sa.template load_lds<EDGE, kScalarBase>(st, kt, wave);
          sb.template load_lds<EDGE, kScalarBase>(st + SA::ELEMS, kt, wave);
        } else {
          V ra[SA::LOADS], rb[SB::LOADS];
          sa.template load<true>(ra, kt);
          sb.template load<true>(rb, kt);
          sa.store(st, ra);
          sb.store(st + SA::ELEMS, rb);
        }
      };
      fill(0);
      if (1 < nkt) fill(1);
      copies_landed_sync();
      T x[4][MB], y[4][MB], xb[4][MB], yb[4][MB];
      fetch_operands<T, BTM, AKC, MB>(smem, wm, 0, lane, x);
      fetch_operands<T, BTN, BKC, MB>(smem + SA::ELEMS, wn, 0, lane, xb);
      // Steady state (tile kt+2 exists and is whole): branch-free, with the
      // LDS reads and copies spread among the MFMAs (sched_group_barrier) so
      // that neither wave on a SIMD sits in a long non-MFMA stretch.
      int kt = 0;
      const int nsteady = (nkt < nkt_whole ? nkt : nkt_whole) - 2;
      for (; kt < nsteady; ++kt) {
        T *cur = smem + (kt & 1) * STAGE;
        const T *nxt = smem + ((kt + 1) & 1) * STAGE;
        fetch_operands<T, BTM, AKC, MB>(cur, wm, 16, lane, y);
        fetch_operands<T, BTN, BKC, MB>(cur + SA::ELEMS, wn, 16, lane, yb);
  #pragma unroll
        for (int s = 0; s < 4; ++s)
  #pragma unroll
          for (int i = 0; i < MB; ++i)
  #pragma unroll
            for (int j = 0; j < MB; ++j) acc[i][j] = Ty<T>::mfma(x[s][i], xb[s][j], acc[i][j]);
  #pragma unroll
        for (int g = 0; g < 2 * MB; ++g) {
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
        }
        // Fences for the scheduler: without them it moves most MFMAs of
        // step 2 past the barrier and the copies of step 4 behind them
        // (measured 127 against 144 TFLOP/s at 8192^3).
        __builtin_amdgcn_sched_barrier(0);
        copies_landed_sync();
        __builtin_amdgcn_sched_barrier(0);
        sa.template load_lds<EDGE, kScalarBase>(cur, kt + 2, wave);
        sb.template load_lds<EDGE, kScalarBase>(cur + SA::ELEMS, kt + 2, wave);
        fetch_operands<T, BTM, AKC, MB>(nxt, wm, 0, lane, x);
        fetch_operands<T, BTN, BKC, MB>(nxt + SA::ELEMS, wn, 0, lane, xb);
  #pragma unroll
        for (int s = 0; s < 4; ++s)
  #pragma unroll
          for (int i = 0; i < MB; ++i)
  #pragma unroll
            for (int j = 0; j < MB; ++j) acc[i][j] = Ty<T>::mfma(y[s][i], yb[s][j], acc[i][j]);
        // The copies go out spread over the MFMAs: a burst of them right
        // after the barrier backs up the L1 and stalls the wave on a copy
        // (a timing-only copy without the steady-state copies ran 2.8%
        // faster). 6 MFMAs per copy (8192^3, A/B on one box: NN 147.9 ->
        // 149.0, NT 147.9 -> 149.0, TT 148.2 -> 149.0; 3 or 4 per copy the
        // same within noise).
        constexpr int kMfmaPerCopy = 6;
  #pragma unroll
        for (int g = 0; g < SA::LOADS + SB::LOADS; ++g) {
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, kMfmaPerCopy, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, 1, 0);
        }
  #pragma unroll
        for (int g = 0; g < 2 * MB; ++g) {
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
        }
      }
      // The last two k-tiles (all of them for edge tiles' short loops).
      for (; kt < nkt; ++kt) {
        T *cur = smem + (kt & 1) * STAGE;
        const T *nxt = smem + ((kt + 1) & 1) * STAGE;
        fetch_operands<T, BTM, AKC, MB>(cur, wm, 16, lane, y);
        fetch_operands<T, BTN, BKC, MB>(cur + SA::ELEMS, wn, 16, lane, yb);
  #pragma unroll
        for (int s = 0; s < 4; ++s)
  #pragma unroll
          for (int i = 0; i < MB; ++i)
  #pragma unroll
            for (int j = 0; j < MB; ++j) acc[i][j] = Ty<T>::mfma(x[s][i], xb[s][j], acc[i][j]);
        copies_landed_sync();
        if (kt + 2 < nkt) fill(kt + 2);
        if (kt + 1 < nkt) {
          fetch_operands<T, BTM, AKC, MB>(nxt, wm, 0, lane, x);
          fetch_operands<T, BTN, BKC, MB>(nxt + SA::ELEMS, wn, 0, lane, xb);
        }
  #pragma unroll
        for (int s = 0; s < 4; ++s)
  #pragma unroll
          for (int i = 0; i < MB; ++i)
  #pragma unroll
            for (int j = 0; j < MB; ++j) acc[i][j] = Ty<T>::mfma(y[s][i], yb[s][j], acc[i][j]);
      }
    } else if constexpr (VEC) {
      // fp64 with 16-byte aligned operands: the same LDS copies, one 16-k
      // chunk per k-tile, operands fetched one MFMA step (4 k) at a time and
      // double buffered across steps. Tile kt, step s: fetch step s+1 (for
      // s = 3: wait for this wave's copies, barrier, copies of tile kt+2
      // into buffer kt&1, fetch step 0 of tile kt+1), then the MFMAs of step
      // s. A copy has a whole k-tile to land; after each barrier the MFMAs of
      // the last step cover the first LDS reads of the next tile.
      static_assert(BK == 16, "the fp64 copy loop assumes one 16-k chunk per k-tile");
      constexpr bool kScalarBase = AKC || BKC;
      const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
      sa.template init_copy<EDGE>();
      sb.template init_copy<EDGE>();
      auto fill = [&](int kt) {
        T *st = smem + (kt & 1) * STAGE;
        if (kt < nkt_whole) {
          sa.template load_lds<EDGE, kScalarBase>(st, kt, wave);
          sb.template load_lds<EDGE, kScalarBase>(st + SA::ELEMS, kt, wave);
        } else {
          V ra[SA::LOADS], rb[SB::LOADS];
          sa.template load<true>(ra, kt);
          sb.template load<true>(rb, kt);
          sa.store(st, ra);
          sb.store(st + SA::ELEMS, rb);
        }
      };
      fill(0);
      if (1 < nkt) fill(1);
      copies_landed_sync();
      T a[2][MB], b[2][MB];
      fetch_step<T, BTM, AKC, MB>(smem, wm, 0, 0, lane, a[0]);
      fetch_step<T, BTN, BKC, MB>(smem + SA::ELEMS, wn, 0, 0, lane, b[0]);
      // One k-tile; TAIL: tile kt+2 may be missing or partial (the last two
      // k-tiles), otherwise it is whole and the loop body is branch-free.
      auto tile = [&](int kt, auto tail_tag) {
        constexpr bool TAIL = decltype(tail_tag)::value;
        T *cur = smem + (kt & 1) * STAGE;
        const T *nxt = smem + ((kt + 1) & 1) * STAGE;
  #pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int u = s & 1, w = u ^ 1;
          if (s < 3) {
            fetch_step<T, BTM, AKC, MB>(cur, wm, 0, s + 1, lane, a[w]);
            fetch_step<T, BTN, BKC, MB>(cur + SA::ELEMS, wn, 0, s + 1, lane, b[w]);
          } else {
            __builtin_amdgcn_sched_barrier(0);
            copies_landed_sync();
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (TAIL) {
              if (kt + 2 < nkt) fill(kt + 2);
            } else {
              sa.template load_lds<EDGE, kScalarBase>(cur, kt + 2, wave);
              sb.template load_lds<EDGE, kScalarBase>(cur + SA::ELEMS, kt + 2, wave);
            }
            if (!TAIL || kt + 1 < nkt) {
              fetch_step<T, BTM, AKC, MB>(nxt, wm, 0, 0, lane, a[w]);
              fetch_step<T, BTN, BKC, MB>(nxt + SA::ELEMS, wn, 0, 0, lane, b[w]);
            }
          }
  #pragma unroll
          for (int i = 0; i < MB; ++i)
  #pragma unroll
            for (int j = 0; j < MB; ++j) acc[i][j] = Ty<T>::mfma(a[u][i], b[u][j], acc[i][j]);
          if constexpr (!TAIL) {
            if (s == 3) {
              // The step after the barrier: one copy after each of its
              // first MFMAs, then the next tile's operand reads one per
              // MFMA. Left to the scheduler the eight copies issued as one
              // burst ahead of the MFMAs, and a copy the L1 could not yet
              // take stalled them (4096^3, A/B on one box: NT 70.4 -> 73.1,
              // NN 69.5 -> 72.2, TN 68.9 -> 72.0, TT 68.8 -> 71.5 TFLOP/s;
              // two MFMAs per copy: 72.8 / 70.9 / 69.5 / 70.7).
  #pragma unroll
              for (int c = 0; c < SA::LOADS + SB::LOADS; ++c) {
                __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
                __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, 1, 0);
              }
  #pragma unroll
              for (int c = 0; c < MB * MB - (SA::LOADS + SB::LOADS); ++c) {
                __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
                __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
              }
            }
          }
        }
      };
      int kt = 0;
      const int nsteady = (nkt < nkt_whole ? nkt : nkt_whole) - 2;
      for (; kt < nsteady; ++kt) tile(kt, std::false_type{});
      for (; kt < nkt; ++kt) tile(kt, std::true_type{});
    } else {
      V ra[SA::LOADS], rb[SB::LOADS];
      if (0 < nkt_whole) {
        sa.template load<false, EDGE>(ra, 0);
        sb.template load<false, EDGE>(rb, 0);
      } else {
        sa.template load<true>(ra, 0);
        sb.template load<true>(rb, 0);
      }
      sa.store(smem, ra);
      sb.store(smem + SA::ELEMS, rb);

      if constexpr (KernelPolicy<T>::kPerStep) {
        __syncthreads();
        for (int kt = 0; kt < nkt; ++kt) {
          const bool more = kt + 1 < nkt;
          if (more) {
            if (kt + 1 < nkt_whole) {
              sa.template load<false, EDGE>(ra, kt + 1);
              sb.template load<false, EDGE>(rb, kt + 1);
            } else {
              sa.template load<true>(ra, kt + 1);
              sb.template load<true>(rb, kt + 1);
            }
          }
          const T *As = smem + (kt & 1) * STAGE;
          const T *Bs = As + SA::ELEMS;
    #pragma unroll
          for (int kc = 0; kc < BK; kc += 16) {
    #pragma unroll
            for (int s = 0; s < 4; ++s) {
              T a[MB], b[MB];
              fetch_step<T, BTM, AKC, MB>(As, wm, kc, s, lane, a);
              fetch_step<T, BTN, BKC, MB>(Bs, wn, kc, s, lane, b);
    #pragma unroll
              for (int i = 0; i < MB; ++i)
    #pragma unroll
                for (int j = 0; j < MB; ++j) acc[i][j] = Ty<T>::mfma(a[i], b[j], acc[i][j]);
            }
          }
          if (more) {
            T *next = smem + ((kt + 1) & 1) * STAGE;
            sa.store(next, ra);
            sb.store(next + SA::ELEMS, rb);
          }
          __syncthreads();
        }
      } else {
        // Two 16-k chunks per k-tile, software pipelined so that LDS reads and
        // global loads are in flight under MFMAs. On entry to iteration kt:
        // X = chunk 0 of tile kt (registers), R = tile kt+1 (registers, loaded
        // one iteration earlier), tile kt in LDS buffer kt&1.
        //   1. LDS reads of chunk 1 of tile kt into Y
        //   2. MFMAs on X
        //   3. R -> LDS buffer (kt+1)&1; global loads of tile kt+2 into R
        //   4. barrier: every wave has finished reading buffer kt&1 (chunk 0
        //      at the end of kt-1, chunk 1 in step 1, both waited for) and has
        //      written tile kt+1, so buffer kt&1 may be refilled in kt+1
        //   5. LDS reads of chunk 0 of tile kt+1 into X
        //   6. MFMAs on Y
        static_assert(BK == 32, "the pipelined fp32 loop assumes two 16-k chunks per k-tile");
        if (1 < nkt) {
          if (1 < nkt_whole) {
            sa.template load<false, EDGE>(ra, 1);
            sb.template load<false, EDGE>(rb, 1);
          } else {
            sa.template load<true>(ra, 1);
            sb.template load<true>(rb, 1);
          }
        }
        __syncthreads();
        T x[4][MB], y[4][MB], xb[4][MB], yb[4][MB];
        fetch_operands<T, BTM, AKC, MB>(smem, wm, 0, lane, x);
        fetch_operands<T, BTN, BKC, MB>(smem + SA::ELEMS, wn, 0, lane, xb);
        // Steady state (both next tiles exist and are whole): the same steps
        // without branches, with the chunk-1 reads, the LDS stores and the
        // global loads spread among the chunk-0 MFMAs (sched_group_barrier:
        // 1 MFMA per read, 3 per store, 2 per global load) so that no wave sits
        // in a long non-MFMA stretch while the other wave on its SIMD is in one
        // too. Measured +5-8% over leaving the order to the scheduler.
        int kt = 0;
        const int nsteady = (nkt < nkt_whole ? nkt : nkt_whole) - 2;
        for (; kt < nsteady; ++kt) {
          const T *As = smem + (kt & 1) * STAGE;
          T *next = smem + ((kt + 1) & 1) * STAGE;
          fetch_operands<T, BTM, AKC, MB>(As, wm, 16, lane, y);
          fetch_operands<T, BTN, BKC, MB>(As + SA::ELEMS, wn, 16, lane, yb);
    #pragma unroll
          for (int s = 0; s < 4; ++s)
    #pragma unroll
            for (int i = 0; i < MB; ++i)
    #pragma unroll
              for (int j = 0; j < MB; ++j) acc[i][j] = Ty<T>::mfma(x[s][i], xb[s][j], acc[i][j]);
          // Stores then loads, operand by operand; with A mn-contiguous and B
          // k-contiguous (NN), B's eight-rows-per-instruction loads go first
          // (measured +3-5% for NN, neutral to slightly negative elsewhere).
          if constexpr (BKC && !AKC) {
            sb.store(next + SA::ELEMS, rb);
            sa.store(next, ra);
            sb.template load<false, EDGE>(rb, kt + 2);
            sa.template load<false, EDGE>(ra, kt + 2);
          } else {
            sa.store(next, ra);
            sb.store(next + SA::ELEMS, rb);
            sa.template load<false, EDGE>(ra, kt + 2);
            sb.template load<false, EDGE>(rb, kt + 2);
          }
    #pragma unroll
          for (int g = 0; g < 2 * MB; ++g) {
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
          }
    #pragma unroll
          for (int g = 0; g < SA::LOADS + SB::LOADS; ++g) {
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 3, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedDsWrite, 1, 0);
          }
    #pragma unroll
          for (int g = 0; g < SA::LOADS + SB::LOADS; ++g) {
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, 1, 0);
          }
          __syncthreads();
          fetch_operands<T, BTM, AKC, MB>(next, wm, 0, lane, x);
          fetch_operands<T, BTN, BKC, MB>(next + SA::ELEMS, wn, 0, lane, xb);
    #pragma unroll
          for (int s = 0; s < 4; ++s)
    #pragma unroll
            for (int i = 0; i < MB; ++i)
    #pragma unroll
              for (int j = 0; j < MB; ++j) acc[i][j] = Ty<T>::mfma(y[s][i], yb[s][j], acc[i][j]);
        }
        // The last two k-tiles (and every k-tile of edge tiles): guarded loads.
        for (; kt < nkt; ++kt) {
          const bool more = kt + 1 < nkt;
          const T *As = smem + (kt & 1) * STAGE;
          fetch_operands<T, BTM, AKC, MB>(As, wm, 16, lane, y);
          fetch_operands<T, BTN, BKC, MB>(As + SA::ELEMS, wn, 16, lane, yb);
    #pragma unroll
          for (int s = 0; s < 4; ++s)
    #pragma unroll
            for (int i = 0; i < MB; ++i)
    #pragma unroll
              for (int j = 0; j < MB; ++j) acc[i][j] = Ty<T>::mfma(x[s][i], xb[s][j], acc[i][j]);
          T *next = smem + ((kt + 1) & 1) * STAGE;
          if (more) {
            sa.store(next, ra);
            sb.store(next + SA::ELEMS, rb);
            if (kt + 2 < nkt) {
              if (kt + 2 < nkt_whole) {
                sa.template load<false, EDGE>(ra, kt + 2);
                sb.template load<false, EDGE>(rb, kt + 2);
              } else {
                sa.template load<true>(ra, kt + 2);
                sb.template load<true>(rb, kt + 2);
              }
            }
          }
          __syncthreads();
          if (more) {
            fetch_operands<T, BTM, AKC, MB>(next, wm, 0, lane, x);
            fetch_operands<T, BTN, BKC, MB>(next + SA::ELEMS, wn, 0, lane, xb);
          }
    #pragma unroll
          for (int s = 0; s < 4; ++s)
    #pragma unroll
            for (int i = 0; i < MB; ++i)
    #pragma unroll
              for (int j = 0; j < MB; ++j) acc[i][j] = Ty<T>::mfma(y[s][i], yb[s][j], acc[i][j]);
        }
      }
    }
  };
  if (interior)
    mainloop(std::integral_constant<bool, false>{});
  else
    mainloop(std::integral_constant<bool, true>{});

  // Epilogue: C = alpha*acc + beta*C on the tile's in-range (and, for
  // sgemmtr/ssyrk, in-triangle) elements.
  if (unit >= 0) {
    // Split-k unit: raw partial sums of the whole BTM x BTN tile; rows and
    // columns past m, n hold sums over clamped operand rows, which
    // split_fixup never stores.
    T *slice = p.ws + (int64_t)unit * BTM * BTN;
    if constexpr (!AKC || sizeof(T) == 4) {
      GemmArgs<T> q = p;
      q.C = slice;
      q.ldc = BTM;
      q.alpha = (T)1;
      q.beta = (T)0;
      epilogue_vec<T, AKC, BKC, MB, MB>(q, acc, wm, wn, lane);
    } else {
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < MB; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            slice[(wm + out_row<T, AKC, MB>(i, q, lane)) +
                  (int64_t)(wn + out_col<BKC, MB, VW>(j, lane)) * BTM] = acc[i][j][q];
    }
    return;
  }
  const T alpha = p.alpha, beta = p.beta;
  const bool tri_diag = p.uplo != 0 && tm == tn;
  if constexpr (!AKC || sizeof(T) == 4) {
    if (interior && !tri_diag && p.c_vec) {
      epilogue_vec<T, AKC, BKC, MB, MB>(p, acc, m0 + wm, n0 + wn, lane);
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < MB; ++i) {
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const int64_t col = n0 + wn + out_col<BKC, MB, VW>(j, lane);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t row = m0 + wm + out_row<T, AKC, MB>(i, q, lane);
        bool ok = row < p.m && col < p.n;
        if (tri_diag) ok = ok && (p.uplo == WGB_LOWER ? row >= col : row <= col);
        if (ok) {
          T *cp = p.C + row + col * p.ldc;
          T v = alpha * acc[i][j][q];
          if (beta != (T)0) v = fma(beta, *cp, v);
          *cp = v;
        }
      }
    }
  }
}


// The instantiations are held to 256 registers (two waves per SIMD)
// explicitly, except the register-staged ones (element-aligned operands)
// other than fp32 TN and, for the paired fp32 kernels and fp64, other than
// those with a k-contiguous operand (their earlier bound, not re-measured). The fp32 kernels whose operands are both k-contiguous or
// both mn-contiguous would fit without the bound too, with accumulators in
// AGPRs; with scalar-base LDS copies the bound measured faster for them (NT
// 8192^3 146.8 -> 148.2 TFLOP/s, ssyrk 8192/4096 140.9 -> 141.9). The
// register-staged kernels ran faster without it except TN (ragged 8191 x
// 8193 x 4097, A/B on one box: NT 130.7 -> 136.5, NN 136.1 -> 138.0, TT
// 133.9 -> 135.5; TN 137.8 -> 135.2).
//
// PAIR (launches with a k band, p.band != kBandNone): a tile row's (or
// column's) k range grows with its index, so block b takes the tile pair
// (r, c) and (tiles-1-r, c) (columns for a band on op(B)) and every block
// does the same work, whatever order the dispatcher fills the CUs in.
//
// K2: the two-part k range of GemmArgs (k-tiles from kt_switch on read A2 and
// B2); no PAIR.
template <typename T, int BT, bool AKC, bool BKC, bool VEC, bool PAIR, bool K2 = false>
__global__ __launch_bounds__(kThreads, (VEC || (AKC && BKC) ||
                                       ((PAIR || sizeof(T) == 8) && (AKC || BKC)))
                                          ? 2
                                          : 1) void gemm_kernel(GemmArgs<T> p) {
  constexpr int BK = 128 / (int)sizeof(T);
  typedef Stager<T, BT, AKC, VEC> SA;
  typedef Stager<T, BT, BKC, VEC> SB;
  constexpr int STAGE = SA::ELEMS + SB::ELEMS;
  __shared__ __attribute__((aligned(16))) T smem[2 * STAGE];

  if constexpr (!PAIR) {
    // Block -> tile and k-range: the first nregular blocks take whole tiles
    // (XCD-remapped), the rest are split-k units of the tail tiles.
    int tm, tn, unit = -1, kt0 = 0;
    const int nkt_all = (int)((p.k + BK - 1) / BK);
    int nkt = nkt_all;
    if ((int)blockIdx.x < p.nregular) {
      logical_tile(xcd_remap(blockIdx.x, p.nregular), p.tiles_m, p.tiles_n, p.uplo, tm, tn);
    } else {
      unit = (int)blockIdx.x - p.nregular;
      logical_tile(p.nregular + unit / p.splits, p.tiles_m, p.tiles_n, p.uplo, tm, tn);
      kt0 = (unit % p.splits) * p.kt_split;
      nkt = nkt_all - kt0 < p.kt_split ? nkt_all - kt0 : p.kt_split;
    }
    // (nkt >= 1: k > 0 here, and the host never plans an empty split; an
    // explicit nkt check costs the fp32 loop ~60 VGPRs of scheduling freedom.)
    if (tm < 0 || tn < 0 || tm >= p.tiles_m || tn >= p.tiles_n) return;  // block-uniform
    gemm_tile<T, BT, BT, kThreads, AKC, BKC, VEC, K2>(p, tm, tn, unit, kt0, nkt, smem, (int)threadIdx.x);
  } else {
    const int nkt_all = (int)((p.k + BK - 1) / BK);
    const bool on_rows = p.band == wgb::kBandALower || p.band == wgb::kBandAUpper;
    const int prs = on_rows ? (p.tiles_m + 1) / 2 : p.tiles_m;
    const int pcs = on_rows ? p.tiles_n : (p.tiles_n + 1) / 2;
    int pr, pc;
    logical_tile(xcd_remap(blockIdx.x, p.nregular), prs, pcs, 0, pr, pc);
#pragma unroll 1
    for (int pass = 0; pass < 2; ++pass) {
      int tm = pr, tn = pc;
      if (pass == 1) {
        if (on_rows)
          tm = p.tiles_m - 1 - pr;
        else
          tn = p.tiles_n - 1 - pc;
        if (tm == pr && tn == pc) break;  // the middle row / column of an odd count
        __syncthreads();  // every wave is done with the first tile's LDS stages
      }
      // op(A) lower: k < m0 + BT; op(A) upper: k >= m0; op(B) lower
      // (nonzero for k >= j): k >= n0; op(B) upper: k < n0 + BT.
      constexpr int TK = BT / BK;
      const int lo = p.band == wgb::kBandAUpper ? tm * TK : p.band == wgb::kBandBLower ? tn * TK : 0;
      int hi = p.band == wgb::kBandALower ? (tm + 1) * TK
                                          : p.band == wgb::kBandBUpper ? (tn + 1) * TK : nkt_all;
      if (hi > nkt_all) hi = nkt_all;
      // threadIdx.x passed through an empty asm each pass: the values the
      // tile derives from it are recomputed per tile instead of being hoisted
      // out of this loop and held in registers across both tiles.
      int t = (int)threadIdx.x;
      asm volatile("" : "+v"(t));
      gemm_tile<T, BT, BT, kThreads, AKC, BKC, VEC, false, true>(p, tm, tn, -1, lo, hi - lo, smem, t);
    }
  }
}

// Wide fp32 tier: 256 x 128 tiles of C, two blocks of 4 waves per CU, each
// wave a 128 x 64 part of the tile (8 x 4 MFMA blocks, 128 accumulator
// registers), k-tiles of 16 floats in a ring of three 24 KB LDS stages
// (72 KB per block), copies issued two k-tiles ahead. Per flop it copies
// 3/4 of the operand bytes of a 128 x 128 tile, and the second block on a
// CU covers each block's epilogue.
constexpr int kWideM = 256, kWideN = 128, kWideBK = 16, kWideStages = 3;

// s_waitcnt immediate (gfx9 encoding): at most n vector-memory operations of
// this wave in flight (vmcnt, bits 3:0 and 15:14), every LDS operation
// complete (lgkmcnt 0), exports not waited for.
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }

// Waits until at most VM of this wave's copies are in flight and its LDS
// reads are done, then joins the block barrier. No memory fence: a fence
// would wait for every copy in flight (vmcnt 0); the empty asm statements
// keep the compiler from moving memory accesses across the barrier and the
// sched_barriers keep the scheduler from moving anything.
template <int VM>
__device__ __forceinline__ void wait_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(VM));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Copies of one operand's BT x 16 k-tile, 256 threads, 16 bytes each:
//   KC (k-contiguous): staged [row][k], 64-byte rows whose four 16-byte
//     chunks sit at chunk ^ ((row >> 2) & 3): a 16-lane read of one chunk of
//     16 consecutive rows then touches every bank once;
//   !KC: staged [k][row], rows of BT floats.
// Thread t's copy r lands at 16 t bytes + r * 4 KB of the operand's stage
// (the LDS DMA address rule), so each thread reads the global vector that
// belongs there.
template <int BT, bool KC>
struct WideStager {
  static constexpr int LOADS = BT / 64;  // 16-byte copies per thread per k-tile
  static constexpr int ELEMS = BT * kWideBK;
  const float *origin;  // k-tile 0 of the tile
  int64_t k_step;       // elements per k-tile
  uint32_t voff[LOADS];
  __device__ void init(const float *P, int64_t ld, int64_t row0, int t) {
    if (KC) {
      origin = P + row0 * ld;
      k_step = kWideBK;
      const int row = t >> 2, pos = t & 3, key = (t >> 4) & 3;
#pragma unroll
      for (int r = 0; r < LOADS; ++r)
        voff[r] = (uint32_t)((((int64_t)(row + 64 * r)) * ld + 4 * (pos ^ key)) * (int64_t)sizeof(float));
    } else {
      origin = P + row0;
      k_step = kWideBK * ld;
      constexpr int VPK = BT / 4, KROWS = 256 / VPK;
      const int mv = t % VPK, kk = t / VPK;
#pragma unroll
      for (int r = 0; r < LOADS; ++r)
        voff[r] = (uint32_t)((((int64_t)(kk + KROWS * r)) * ld + 4 * mv) * (int64_t)sizeof(float));
    }
  }
  // The wave-uniform tile origin of k-tile kt.
  __device__ const char *base(int kt) const {
    const uint64_t o64 = (uint64_t)(origin + (int64_t)kt * k_step);
    uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)o64);
    uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(o64 >> 32));
    asm volatile("" : "+s"(lo), "+s"(hi));
    return (const char *)(((uint64_t)hi << 32) | lo);
  }
  // Copy r of this thread from origin o into its operand stage.
  __device__ void copy_one(const char *o, float *stage, int wave, int r) const {
    uint32_t v = voff[r];
    asm volatile("" : "+v"(v));
    copy16_to_lds(o + v, stage + wave * 256 + r * 1024);
  }
  __device__ void copy(float *stage, int kt, int wave) const {
    const char *o = base(kt);
#pragma unroll
    for (int r = 0; r < LOADS; ++r) copy_one(o, stage, wave, r);
  }
};

// MFMA operands of one 16-k tile for MB 16-row blocks from rows wrow.. of
// a wide stage (the k order and row placement of fetch_operands).
template <int BT, bool KC, int MB>
__device__ __forceinline__ void wide_operands(const float *stage, int wrow, int lane,
                                              float (&out)[4][MB]) {
  typedef float V4 __attribute__((ext_vector_type(4)));
  const int g = lane >> 4, i16 = lane & 15;
  if (KC) {
    const int pos = g ^ ((i16 >> 2) & 3);
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      V4 v = *reinterpret_cast<const V4 *>(stage + (wrow + 16 * b + i16) * kWideBK + 4 * pos);
#pragma unroll
      for (int s = 0; s < 4; ++s) out[s][b] = v[s];
    }
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int h = 0; h < MB / 4; ++h) {
        V4 v = *reinterpret_cast<const V4 *>(stage + (4 * g + s) * BT + wrow + 64 * h + 4 * i16);
#pragma unroll
        for (int c = 0; c < 4; ++c) out[s][4 * h + c] = v[c];
      }
  }
}

// Read `idx` of wide_operands' reads (KC: block idx; !KC: step idx / (MB / 4),
// row group idx % (MB / 4)), so reads can be placed one by one.
template <int BT, bool KC, int MB>
__device__ __forceinline__ void wide_read(const float *stage, int wrow, int lane, float (&out)[4][MB],
                                          int idx) {
  typedef float V4 __attribute__((ext_vector_type(4)));
  const int g = lane >> 4, i16 = lane & 15;
  if (KC) {
    const int pos = g ^ ((i16 >> 2) & 3);
    V4 v = *reinterpret_cast<const V4 *>(stage + (wrow + 16 * idx + i16) * kWideBK + 4 * pos);
#pragma unroll
    for (int s = 0; s < 4; ++s) out[s][idx] = v[s];
  } else {
    const int s = idx / (MB / 4), h = idx % (MB / 4);
    V4 v = *reinterpret_cast<const V4 *>(stage + (4 * g + s) * BT + wrow + 64 * h + 4 * i16);
#pragma unroll
    for (int c = 0; c < 4; ++c) out[s][4 * h + c] = v[c];
  }
}

// v_mfma_f32_16x16x4f32 with the accumulator pinned in AGPRs. Left to the
// builtin at two waves per SIMD, the compiler either took the VGPR form and
// spilled or kept its AGPRs as spill space (100-230 v_accvgpr moves per
// k-tile pair). Being volatile, these statements also keep the memory
// operations between them where the source puts them.
__device__ __forceinline__ void mfma_agpr(Ty<float>::acc &c, float a, float b) {
  asm volatile("v_mfma_f32_16x16x4_f32 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}

// The host launches it only with m % 256 == 0, n % 128 == 0, k a multiple
// of 16 with at least 3 k-tiles, 16-byte aligned operands with 32-bit copy
// offsets, a vector-aligned C, full C (no triangle, band or split). Measured
// at 8192^3 on MI355X against the 128 x 128 tier (A/B, one box): NN 148.9
// -> 151.3, NT 148.9 -> 150.2, TN 148.9 -> 150.0, TT 148.4 -> 150.3
// TFLOP/s; timing-only variants put its copies at ~1.5% (2.8% in the 128
// tier) and its epilogue at ~0.6%.
template <bool AKC, bool BKC>
__global__ __launch_bounds__(kThreads, 2) void gemm_wide_kernel(GemmArgs<float> p) {
  typedef float T;
  typedef Ty<T>::acc Acc;
  constexpr int MA = kWideM / 32, MN = kWideN / 32;
  typedef WideStager<kWideM, AKC> SA;
  typedef WideStager<kWideN, BKC> SB;
  constexpr int STAGE = SA::ELEMS + SB::ELEMS;
  constexpr int NCOPY = SA::LOADS + SB::LOADS;  // copies per thread per k-tile
  __shared__ __attribute__((aligned(16))) T smem[kWideStages * STAGE];

  int tm, tn;
  logical_tile(xcd_remap((int)blockIdx.x, p.ntiles), p.tiles_m, p.tiles_n, 0, tm, tn);
  const int t = (int)threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = (wave & 1) * (kWideM / 2), wn = (wave >> 1) * (kWideN / 2);
  SA sa;
  SB sb;
  sa.init(p.A, p.lda, (int64_t)tm * kWideM, t);
  sb.init(p.B, p.ldb, (int64_t)tn * kWideN, t);
  const int nkt = (int)(p.k / kWideBK);
  auto copy = [&](T *st, int kt) {
    sa.copy(st, kt, wave);
    sb.copy(st + SA::ELEMS, kt, wave);
  };
  Acc acc[MA][MN];
#pragma unroll
  for (int i = 0; i < MA; ++i)
#pragma unroll
    for (int j = 0; j < MN; ++j) acc[i][j] = Acc(0);
  // One copy per 8 MFMAs (5 and 3 measured slower, 10 the same).
  constexpr int kMfmaPerCopy = 8;
  static_assert(kMfmaPerCopy * NCOPY <= 2 * MA * MN, "copies fit in half a k-tile");
  // MFMA q (0..63) of half h of a k-tile: k-step 2h + q / 32, block (i, j) =
  // ((q % 32) / MN, q % MN); an accumulator recurs every 32 MFMAs.
  auto mf = [&](const T (&a)[4][MA], const T (&b)[4][MN], int h, int q) {
    const int st = 2 * h + q / 32, i = (q % 32) / MN, j = q % MN;
    mfma_agpr(acc[i][j], a[st][i], b[st][j]);
  };
  // First half of a k-tile: k-steps 0-1, one copy of k-tile ckt into stage
  // cst after every kMfmaPerCopy MFMAs.
  auto half0 = [&](const T (&a)[4][MA], const T (&b)[4][MN], T *cst, int ckt) {
    ckt = ckt < nkt ? ckt : nkt - 1;
    const char *oa = sa.base(ckt), *ob = sb.base(ckt);
#pragma unroll
    for (int q = 0; q < 64; ++q) {
      mf(a, b, 0, q);
      if (q % kMfmaPerCopy == kMfmaPerCopy - 1 && q / kMfmaPerCopy < NCOPY) {
        const int r = q / kMfmaPerCopy;
        if (r < SA::LOADS)
          sa.copy_one(oa, cst, wave, r);
        else
          sb.copy_one(ob, cst + SA::ELEMS, wave, r - SA::LOADS);
      }
    }
  };
  // Second half: k-steps 2-3, the next k-tile's 12 operand reads from stage
  // rst after the first 12 MFMAs, one per MFMA.
  auto half1 = [&](const T (&a)[4][MA], const T (&b)[4][MN], const T *rst, T (&na)[4][MA],
                   T (&nb)[4][MN]) {
#pragma unroll
    for (int q = 0; q < 64; ++q) {
      mf(a, b, 1, q);
      if (q < MA)
        wide_read<kWideM, AKC, MA>(rst, wm, lane, na, q);
      else if (q < MA + MN)
        wide_read<kWideN, BKC, MN>(rst + SA::ELEMS, wn, lane, nb, q - MA);
    }
  };
  // Paired form, for two k-contiguous operands: the second half of an even
  // k-tile issues the copies of the next two k-tiles, each copy of one beside
  // the same rows' copy of the other, so both 64-byte halves of each 128-byte
  // line are fetched together. With one k-tile per half, the second half of
  // a line was read a whole k-tile after the first and had mostly left L2
  // (rows 32 KB apart at 8192^3): TN fetched 16.9x its algorithmic bytes
  // from HBM, paired 10.4x, at the same speed. For one k-contiguous operand
  // (NN, TT) pairing cost 0.3-0.6% and did not cut TT's 8.2x.
  constexpr bool kPairCopies = AKC && BKC;
  auto half1p = [&](const T (&a)[4][MA], const T (&b)[4][MN], const T *rst, T (&na)[4][MA],
                    T (&nb)[4][MN], T *c2, int k2, T *c3, int k3) {
    k2 = k2 < nkt ? k2 : nkt - 1;
    k3 = k3 < nkt ? k3 : nkt - 1;
    const char *oa2 = sa.base(k2), *ob2 = sb.base(k2), *oa3 = sa.base(k3), *ob3 = sb.base(k3);
#pragma unroll
    for (int q = 0; q < 64; ++q) {
      mf(a, b, 1, q);
      if (q < MA) {
        wide_read<kWideM, AKC, MA>(rst, wm, lane, na, q);
      } else if (q < MA + MN) {
        wide_read<kWideN, BKC, MN>(rst + SA::ELEMS, wn, lane, nb, q - MA);
      } else if ((q - (MA + MN)) % 4 == 3 && (q - (MA + MN)) / 4 < 2 * NCOPY) {
        const int c = (q - (MA + MN)) / 4, r = c / 2;
        T *cst = (c & 1) ? c3 : c2;
        if (r < SA::LOADS)
          sa.copy_one((c & 1) ? oa3 : oa2, cst, wave, r);
        else
          sb.copy_one((c & 1) ? ob3 : ob2, cst + SA::ELEMS, wave, r - SA::LOADS);
      }
    }
  };
  auto half0n = [&](const T (&a)[4][MA], const T (&b)[4][MN]) {
#pragma unroll
    for (int q = 0; q < 64; ++q) mf(a, b, 0, q);
  };

  copy(smem, 0);
  copy(smem + STAGE, 1);
  wait_barrier<NCOPY>();
  T x[4][MA], xb[4][MN], y[4][MA], yb[4][MN];
  wide_operands<kWideM, AKC, MA>(smem, wm, lane, x);
  wide_operands<kWideN, BKC, MN>(smem + SA::ELEMS, wn, lane, xb);
  // Two k-tiles per iteration (x / xb, then y / yb). For k-tile kt, with
  // its operands in registers and k-tile kt + 1 in flight or landed:
  //   copies of k-tile kt + 2 into its stage (which held k-tile kt - 1,
  //   whose reads every wave finished before the previous barrier) under
  //   the MFMAs of k-steps 0-1 of k-tile kt;
  //   wait for k-tile kt + 1 (k-tile kt + 2 may still be in flight),
  //   barrier, its operands read into the other registers under the MFMAs
  //   of k-steps 2-3.
  // Copies past the last k-tile re-copy it (a valid address) into a stage
  // nobody reads again, so every iteration is the same branch-free code.
  int s0 = 0, kt = 0;
  for (; kt + 1 < nkt; kt += 2) {
    const int s1 = s0 == 2 ? 0 : s0 + 1, s2 = s1 == 2 ? 0 : s1 + 1;
    if constexpr (kPairCopies) {
      half0n(x, xb);
      wait_barrier<0>();  // k-tile kt + 1 (its copies went out three halves ago)
      half1p(x, xb, smem + s1 * STAGE, y, yb, smem + s2 * STAGE, kt + 2, smem + s0 * STAGE, kt + 3);
      half0n(y, yb);
      wait_barrier<1>();  // k-tile kt + 2 (only k-tile kt + 3's last copy may be in flight)
      half1(y, yb, smem + s2 * STAGE, x, xb);
    } else {
      half0(x, xb, smem + s2 * STAGE, kt + 2);
      wait_barrier<NCOPY>();
      half1(x, xb, smem + s1 * STAGE, y, yb);
      half0(y, yb, smem + s0 * STAGE, kt + 3);
      wait_barrier<NCOPY>();
      half1(y, yb, smem + s2 * STAGE, x, xb);
    }
    s0 = s2;
  }
  if (kt < nkt) {  // an odd k-tile count's last k-tile
#pragma unroll
    for (int q = 0; q < 128; ++q) mf(x, xb, q / 64, q % 64);
  }
  // The accumulators are read next, by instructions the compiler places
  // without knowing the asm statements were MFMAs: wait out the last ones
  // (32 wait states cover an 8-pass MFMA's result), in statements that also
  // redefine every accumulator, so each later read depends on them.
  static_assert(MA * MN == 32, "four groups of eight accumulators");
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
               : "+a"(acc[0][0]), "+a"(acc[0][1]), "+a"(acc[0][2]), "+a"(acc[0][3]),
                 "+a"(acc[1][0]), "+a"(acc[1][1]), "+a"(acc[1][2]), "+a"(acc[1][3]));
#pragma unroll
  for (int i = 2; i < MA; i += 2)
    asm volatile("" : "+a"(acc[i][0]), "+a"(acc[i][1]), "+a"(acc[i][2]), "+a"(acc[i][3]),
                      "+a"(acc[i + 1][0]), "+a"(acc[i + 1][1]), "+a"(acc[i + 1][2]), "+a"(acc[i + 1][3]));
  // No copy may land in LDS after the block has ended.
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  epilogue_vec<T, AKC, BKC, MA, MN, true>(p, acc, (int64_t)tm * kWideM + wm,
                                          (int64_t)tn * kWideN + wn, lane);
}

// Small GEMMs (a few hundred 32x32 tiles of C, k <= kSmallMaxK): one block
// of 16 waves per 32x32 tile, the waves splitting k (wave w takes the 16-k
// chunks w, w+16, ..., CPW of them), each wave loading all its operands
// straight from global memory into MFMA operand registers up front (no LDS
// staging, one memory latency), the 16 partial tiles then added in wave
// order through LDS. One launch and no split-k workspace, where the tiled
// kernels would need a split-k launch plus its fixup to fill the chip.
constexpr int kSmallTile = 32;
constexpr int kSmallWaves = 16;
constexpr int64_t kSmallMaxK = 1024;  // 16 waves x 4 chunks x 16 k

// MFMA operands of one 16-k chunk (k0 .. k0+15) for the two 16-row blocks
// of rows r0 .. r0+31 of op(X), in the k order and row placement of
// fetch_operands (step s of lane group g takes k = k0 + 4g + s; an
// mn-contiguous operand puts rows r0 + 2 i16 + c in block c). Rows past
// `rows` read row rows-1 (their results are never stored); k past K reads 0.
// WHOLE: every k of the chunk is in range and so are all 32 rows.
template <bool KC, bool WHOLE>
__device__ __forceinline__ void small_operands(const float *P, int64_t ld, int64_t rows, int64_t r0,
                                               int64_t K, int64_t k0, int lane, float (&out)[4][2]) {
  typedef float F4 __attribute__((ext_vector_type(4), aligned(4)));
  typedef float F2 __attribute__((ext_vector_type(2), aligned(4)));
  const int g = lane >> 4, i16 = lane & 15;
  if constexpr (KC) {
    const int64_t kk = k0 + 4 * g;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      int64_t row = r0 + 16 * b + i16;
      if (!WHOLE) row = row < rows ? row : rows - 1;
      F4 v;
      if (WHOLE) {
        v = *reinterpret_cast<const F4 *>(P + row * ld + kk);
      } else {
        // k = kk + c for c < nv is in range; every other lane element reads
        // k = min(kk, K - 1) (inside the row) and is replaced by 0: clamped
        // addresses and selects, no branches
        const int64_t nv = K - kk;
        const float *q = P + row * ld + (kk < K ? kk : K - 1);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float x = q[c < nv ? c : 0];
          v[c] = (c < nv) ? x : 0.f;
        }
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) out[s][b] = v[s];
    }
  } else {
    int64_t row = r0 + 2 * i16;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int64_t kk = k0 + 4 * g + s;
      F2 v;
      if (WHOLE) {
        v = *reinterpret_cast<const F2 *>(P + row + kk * ld);
      } else {
        const int64_t kc = kk < K ? kk : K - 1;
        const int64_t ra = row < rows ? row : rows - 1, rb = row + 1 < rows ? row + 1 : rows - 1;
        const float x0 = P[ra + kc * ld], x1 = P[rb + kc * ld];
        v[0] = kk < K ? x0 : 0.f;
        v[1] = kk < K ? x1 : 0.f;
      }
      out[s][0] = v[0];
      out[s][1] = v[1];
    }
  }
}

template <bool AKC, bool BKC, int CPW>
__global__ __launch_bounds__(64 * kSmallWaves) void gemm_small_kernel(GemmArgs<float> p) {
  constexpr int MB = 2;
  typedef Ty<float>::acc Acc;
  __shared__ float red[kSmallWaves][kSmallTile][kSmallTile + 1];  // [wave][col][row]
  const int t = (int)threadIdx.x, lane = t & 63, wave = t >> 6;
  const int tm = (int)blockIdx.x % p.tiles_m, tn = (int)blockIdx.x / p.tiles_m;
  const int64_t m0 = (int64_t)tm * kSmallTile, n0 = (int64_t)tn * kSmallTile;
  const bool inside = m0 + kSmallTile <= p.m && n0 + kSmallTile <= p.n;  // block-uniform
  const int64_t nwhole = p.k / 16;
  float a[CPW][4][2], b[CPW][4][2];
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    // chunks past the end of k load zeros (the guarded form)
    const int64_t c = wave + (int64_t)kSmallWaves * i;
    if (inside && c < nwhole) {
      small_operands<AKC, true>(p.A, p.lda, p.m, m0, p.k, 16 * c, lane, a[i]);
      small_operands<BKC, true>(p.B, p.ldb, p.n, n0, p.k, 16 * c, lane, b[i]);
    } else {
      small_operands<AKC, false>(p.A, p.lda, p.m, m0, p.k, 16 * c, lane, a[i]);
      small_operands<BKC, false>(p.B, p.ldb, p.n, n0, p.k, 16 * c, lane, b[i]);
    }
  }
  Acc acc[MB][MB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[i][j] = Acc(0.f);
#pragma unroll
  for (int c = 0; c < CPW; ++c)
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < MB; ++j) acc[i][j] = Ty<float>::mfma(a[c][s][i], b[c][s][j], acc[i][j]);
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        red[wave][out_col<BKC, MB, 4>(j, lane)][out_row<float, AKC, MB>(i, q, lane)] = acc[i][j][q];
  __syncthreads();
  // one C element per thread: 1024 threads, 32x32 tile
  const int r = t % kSmallTile, cl = t / kSmallTile;
  const int64_t row = m0 + r, col = n0 + cl;
  if (row >= p.m || col >= p.n) return;
  float sum = red[0][cl][r];
#pragma unroll
  for (int w = 1; w < kSmallWaves; ++w) sum += red[w][cl][r];
  float *cp = p.C + row + col * p.ldc;
  float v = p.alpha * sum;
  if (p.beta != 0.f) v = fmaf(p.beta, *cp, v);
  *cp = v;
}

template <bool AKC, bool BKC>
const void *small_kernel_for(int64_t k) {
  const int64_t nch = (k + 15) / 16;
  if (nch <= kSmallWaves) return reinterpret_cast<const void *>(gemm_small_kernel<AKC, BKC, 1>);
  if (nch <= 2 * kSmallWaves) return reinterpret_cast<const void *>(gemm_small_kernel<AKC, BKC, 2>);
  return reinterpret_cast<const void *>(gemm_small_kernel<AKC, BKC, 4>);
}

// C <- beta*C (or 0 when beta == 0) on the uplo part of the m x n C: the
// alpha == 0 / k == 0 path, which reads neither A nor B.
template <typename T>
__global__ void scale_kernel(int64_t m, int64_t n, T beta, T *C, int64_t ldc, int uplo) {
  for (int64_t col = blockIdx.y; col < n; col += gridDim.y) {
    for (int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; row < m;
         row += (int64_t)gridDim.x * blockDim.x) {
      if (uplo == WGB_LOWER && row < col) continue;
      if (uplo == WGB_UPPER && row > col) continue;
      T *cp = C + row + col * ldc;
      *cp = beta == (T)0 ? (T)0 : beta * *cp;
    }
  }
}

// Split-k fixup: C = alpha * (sum over splits, in split order) + beta * C on
// the in-range, in-triangle elements of the tail tiles. A block covers 8
// columns of one tile; a thread takes 4 consecutive rows of one column and
// issues the loads of every split (at most 16) before adding them in split
// order, so the sums are those of a split-by-split loop.
constexpr int kFixupCols = 8;
template <typename T, int BT>
__global__ __launch_bounds__(kFixupCols * BT / 4) void split_fixup(GemmArgs<T> p) {
  typedef T V4 __attribute__((ext_vector_type(4)));
  constexpr int kMaxSplits = 16;
  constexpr int RG = BT / 4;  // row groups per column
  const int per_tile = BT / kFixupCols;
  const int tile = (int)blockIdx.x / per_tile;
  const int cl = ((int)blockIdx.x % per_tile) * kFixupCols + (int)threadIdx.x / RG;
  const int rl = 4 * ((int)threadIdx.x % RG);
  int tm, tn;
  logical_tile(p.nregular + tile, p.tiles_m, p.tiles_n, p.uplo, tm, tn);
  const int64_t row0 = (int64_t)tm * BT + rl, col = (int64_t)tn * BT + cl;
  if (row0 >= p.m || col >= p.n) return;
  const T *src = p.ws + (int64_t)tile * p.splits * BT * BT + (int64_t)cl * BT + rl;
  V4 part[kMaxSplits];
#pragma unroll
  for (int s = 0; s < kMaxSplits; ++s)
    if (s < p.splits) part[s] = *reinterpret_cast<const V4 *>(src + (int64_t)s * BT * BT);
  V4 sum = part[0];
#pragma unroll
  for (int s = 1; s < kMaxSplits; ++s)
    if (s < p.splits) sum += part[s];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t row = row0 + q;
    if (row >= p.m) break;
    if (p.uplo == WGB_LOWER && row < col) continue;
    if (p.uplo == WGB_UPPER && row > col) continue;
    T *cp = p.C + row + col * p.ldc;
    T v = p.alpha * sum[q];
    if (p.beta != (T)0) v = fma(p.beta, *cp, v);
    *cp = v;
  }
}

template <typename T>
using KernelFn = void (*)(GemmArgs<T>);

template <typename T, int BT, bool PAIR>
KernelFn<T> pick_layout(bool akc, bool bkc, bool vec) {
  if (vec) {
    if (akc) return bkc ? gemm_kernel<T, BT, true, true, true, PAIR> : gemm_kernel<T, BT, true, false, true, PAIR>;
    return bkc ? gemm_kernel<T, BT, false, true, true, PAIR> : gemm_kernel<T, BT, false, false, true, PAIR>;
  }
  if (akc) return bkc ? gemm_kernel<T, BT, true, true, false, PAIR> : gemm_kernel<T, BT, true, false, false, PAIR>;
  return bkc ? gemm_kernel<T, BT, false, true, false, PAIR> : gemm_kernel<T, BT, false, false, false, PAIR>;
}

// Banded (paired-tile) kernels serve strmm / dtrmm. Two-part k kernels
// (ssyr2k / dsyr2k) exist for 16-byte aligned operands in the layouts
// op(A) op(B)^T (both mn-contiguous) and op(A)^T op(B) (both k-contiguous):
// the host plans one only there.
template <typename T, int BT>
KernelFn<T> pick_kernel(bool akc, bool bkc, bool vec, bool pair, bool k2) {
  if (k2) return akc ? gemm_kernel<T, BT, true, true, true, false, true>
                     : gemm_kernel<T, BT, false, false, true, false, true>;
  if (pair) return pick_layout<T, BT, true>(akc, bkc, vec);
  return pick_layout<T, BT, false>(akc, bkc, vec);
}

// Resident blocks per CU of one kernel instantiation (LDS and registers),
// cached per (tier, operand layout) slot; 0 = not yet queried.
template <typename T, int BT>
int blocks_per_cu(KernelFn<T> fn, int slot) {
  static int cache[32] = {0};
  if (cache[slot] == 0) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void *>(fn),
                                                     kThreads, 0) != hipSuccess || nb < 1)
      nb = 1;
    cache[slot] = nb;
  }
  return cache[slot];
}

// Grows the context's split-k workspace to at least `bytes`. The stream is
// drained first: an earlier launch may still read the old buffer.
int ensure_workspace(wgb_ctx *ctx, size_t bytes) {
  if (ctx->gemm_ws_bytes >= bytes) return WGB_OK;
  const size_t round = (size_t)16 << 20;
  bytes = (bytes + round - 1) / round * round;
  WGB_CHECK_HIP(hipStreamSynchronize(ctx->stream));
  if (ctx->gemm_ws) WGB_CHECK_HIP(hipFree(ctx->gemm_ws));
  ctx->gemm_ws = nullptr;
  ctx->gemm_ws_bytes = 0;
  if (hipMalloc(&ctx->gemm_ws, bytes) != hipSuccess) {
    (void)hipGetLastError();
    ctx->gemm_ws = nullptr;
    return wgb::fail(WGB_ERR_ALLOC, "hipMalloc of the GEMM split-k workspace failed");
  }
  ctx->gemm_ws_bytes = bytes;
  return WGB_OK;
}

// Where a launch's split-k partials go: ptr == nullptr grows the context's
// workspace (ctx->gemm_ws) with hipMalloc as needed; otherwise a fixed
// buffer of `bytes` that a launch needing more rejects.
struct WsSource {
  void *ptr = nullptr;
  size_t bytes = 0;
};

// Launches one GEMM on a BT tier. Tiles fill `slots` = CUs x resident blocks
// per round; when at least one full round precedes a last round that is at
// most half full, and the tiles have at least 32 k-tiles, the last round's
// tiles are split along k into up to 16 units (at least 4 k-tiles each) so
// that round is as full as the rest, and split_fixup combines the partials
// in split order. A launch of one partial round, or a short k, runs
// unsplit: the fixup rereads and rewrites every tail tile through HBM, which
// cost more than the idle slots did (measured: 1024^3 77 against 61
// TFLOP/s split, 1024 x 4096 x 1024 102 against 89, strsm 4096 69 against
// 61). The partials of rem tail tiles in S splits take rem * S <= slots
// tiles of workspace.
template <typename T, int BT>
int launch_tier(wgb_ctx *ctx, GemmArgs<T> &a, bool akc, bool bkc, bool vec, WsSource wsrc) {
  constexpr int BK = 128 / (int)sizeof(T);
  const bool pair = a.band != wgb::kBandNone;
  const bool k2 = a.kt_switch < (int)((a.k + BK - 1) / BK);
  KernelFn<T> fn = pick_kernel<T, BT>(akc, bkc, vec, pair, k2);
  const int64_t cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
  const int64_t slots = cus * blocks_per_cu<T, BT>(fn, (k2 ? 16 : 0) + (pair ? 8 : 0) + (akc ? 4 : 0) +
                                                           (bkc ? 2 : 0) + (vec ? 1 : 0));
  const int64_t nkt = (a.k + BK - 1) / BK;
  a.nregular = a.ntiles;
  if (pair) {
    // one block per tile pair (rows r and tiles_m-1-r, or columns), no split
    const bool on_rows = a.band == wgb::kBandALower || a.band == wgb::kBandAUpper;
    a.nregular = on_rows ? (a.tiles_m + 1) / 2 * a.tiles_n : a.tiles_m * ((a.tiles_n + 1) / 2);
  }
  a.splits = 1;
  a.kt_split = (int)nkt;
  a.ws = nullptr;
  const int64_t rem = a.ntiles % slots;
  if (a.band == wgb::kBandNone && a.ntiles > slots && rem > 0 && 2 * rem <= slots && nkt >= 32) {
    int64_t S = slots / rem;
    if (S > 16) S = 16;
    if (S > nkt / 4) S = nkt / 4;
    if (S >= 2) {
      const int64_t kts = (nkt + S - 1) / S;
      S = (nkt + kts - 1) / kts;  // every split non-empty
      const size_t need = (size_t)(rem * S) * BT * BT * sizeof(T);
      if (wsrc.ptr) {
        if (need > wsrc.bytes)
          return wgb::fail(WGB_ERR_INVALID_VALUE,
                           "the split-k tail of this problem needs " + std::to_string(need) +
                               " bytes of workspace; the allocation-free entry point holds " +
                               std::to_string(wsrc.bytes));
      } else {
        int st = ensure_workspace(ctx, need);
        if (st) return st;
      }
      a.nregular = (int)(a.ntiles - rem);
      a.splits = (int)S;
      a.kt_split = (int)kts;
      a.ws = static_cast<T *>(wsrc.ptr ? wsrc.ptr : ctx->gemm_ws);
    }
  }
  const int64_t grid = pair ? a.nregular : a.nregular + (int64_t)(a.ntiles - a.nregular) * a.splits;
  void *args[] = {&a};
  WGB_CHECK_HIP(hipLaunchKernel(reinterpret_cast<const void *>(fn), dim3((unsigned)grid),
                                dim3(kThreads), args, 0, ctx->stream));
  if (a.splits > 1) {
    split_fixup<T, BT><<<(unsigned)((a.ntiles - a.nregular) * (BT / kFixupCols)), kFixupCols * BT / 4, 0,
                         ctx->stream>>>(a);
    WGB_CHECK_LAUNCH("split_fixup");
  }
  return WGB_OK;
}

using wgb::aligned16;

int64_t imax(int64_t a, int64_t b) { return a > b ? a : b; }

int check_gemm_args(int uplo, bool want_uplo, int transA, int transB, int64_t m, int64_t n,
                    int64_t k, const void *A, int64_t lda, const void *B, int64_t ldb,
                    const void *C, int64_t ldc) {
  using wgb::fail;
  if (want_uplo && uplo != WGB_LOWER && uplo != WGB_UPPER)
    return fail(WGB_ERR_INVALID_VALUE, "uplo must be WGB_LOWER or WGB_UPPER");
  if (transA != WGB_NO_TRANS && transA != WGB_TRANS)
    return fail(WGB_ERR_INVALID_VALUE, "transA must be WGB_NO_TRANS or WGB_TRANS");
  if (transB != WGB_NO_TRANS && transB != WGB_TRANS)
    return fail(WGB_ERR_INVALID_VALUE, "transB must be WGB_NO_TRANS or WGB_TRANS");
  if (m < 0 || n < 0 || k < 0) return fail(WGB_ERR_INVALID_VALUE, "m, n, and k must be non-negative");
  if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX)
    return fail(WGB_ERR_INVALID_VALUE, "m, n, and k must be below 2^31");
  // Column-major: A is m x k (no-transpose) or k x m (transpose).
  int64_t a_rows = transA == WGB_NO_TRANS ? m : k;
  int64_t b_rows = transB == WGB_NO_TRANS ? k : n;
  if (lda < imax(1, a_rows)) return fail(WGB_ERR_INVALID_VALUE, "lda must be >= max(1, rows of A)");
  if (ldb < imax(1, b_rows)) return fail(WGB_ERR_INVALID_VALUE, "ldb must be >= max(1, rows of B)");
  if (ldc < imax(1, m)) return fail(WGB_ERR_INVALID_VALUE, "ldc must be >= max(1, m)");
  if (m > 0 && n > 0) {
    if (!C) return fail(WGB_ERR_INVALID_VALUE, "C is null");
    if (k > 0 && (!A || !B)) return fail(WGB_ERR_INVALID_VALUE, "A or B is null");
  }
  return WGB_OK;
}

// Enqueues one GEMM (no argument checks, no timing events). With A2 / B2:
// C = alpha (op(A) op(B) + op(A2) op(B2)) + beta C, the second pair at lda /
// ldb with the same transposes (ssyr2k / dsyr2k): one launch over a two-part
// k range when both pairs are 16-byte aligned, k is whole k-tiles and op(A),
// op(B) are both mn-contiguous or both k-contiguous; otherwise two launches,
// the second with beta = 1.
template <typename T>
int gemm_launch(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t m, int64_t n, int64_t k,
                T alpha, const T *A, int64_t lda, const T *B, int64_t ldb, T beta, T *C,
                int64_t ldc, int band, WsSource wsrc = WsSource(), const T *A2 = nullptr,
                const T *B2 = nullptr, const T *side = nullptr) {
  if (m == 0 || n == 0) return WGB_OK;
  if (alpha == (T)0 || k == 0) {
    dim3 block(256);
    int64_t gx = (m + 255) / 256;
    dim3 grid((unsigned)(gx > 1024 ? 1024 : gx), (unsigned)(n > 65535 ? 65535 : n));
    scale_kernel<T><<<grid, block, 0, ctx->stream>>>(m, n, beta, C, ldc, uplo);
    WGB_CHECK_LAUNCH("scale_kernel");
    return WGB_OK;
  }
  GemmArgs<T> a;
  a.m = m;
  a.n = n;
  a.k = k;
  a.alpha = alpha;
  a.beta = beta;
  a.A = A;
  a.lda = lda;
  a.B = B;
  a.ldb = ldb;
  a.C = C;
  a.ldc = ldc;
  a.uplo = uplo;
  a.band = band;
  a.A2 = nullptr;
  a.B2 = nullptr;
  a.kt_switch = INT32_MAX;
  a.band_side = 0;
  if (side && band != wgb::kBandNone) {
    // the banded operand's diagonal blocks from `side` (same ld), the rest in place
    const bool on_a = band == wgb::kBandALower || band == wgb::kBandAUpper;
    a.band_side = 1;
    a.A2 = on_a ? side : nullptr;
    a.B2 = on_a ? nullptr : side;
  }
  const int VW = Ty<T>::VW;
  // Interior tiles store C in vectors of consecutive rows. fp32 does so for
  // any C (a 16-byte store needs dword alignment only, as the loads do);
  // element-wise stores cost about four times the bytes in partial lines
  // (config 3's ragged C, ldc = 8193: 1.1 GB written per NN / NT launch
  // for 0.27 GB of C). fp64 keeps vectors for 16-byte aligned C.
  const bool c_aligned = (ldc % VW == 0) && aligned16(C);
  a.c_vec = sizeof(T) == 4 || c_aligned;
  const bool akc = transA == WGB_TRANS;
  const bool bkc = transB == WGB_NO_TRANS;
  const int64_t fill = ctx->num_cus > 0 ? ctx->num_cus : 256;
  if constexpr (sizeof(T) == 4) {
    // Small problems: below half a launch of 64-tiles the tiled kernels need
    // split-k and a fixup launch; one 32x32 tile per block with k split
    // across its waves does it in one launch.
    const int64_t t32m = (m + kSmallTile - 1) / kSmallTile, t32n = (n + kSmallTile - 1) / kSmallTile;
    const int64_t t64 = ((m + 63) / 64) * ((n + 63) / 64);
    if (uplo == 0 && band == wgb::kBandNone && !A2 && k <= kSmallMaxK && 2 * t64 < fill &&
        t32m * t32n <= 4 * fill) {
      a.tiles_m = (int)t32m;
      a.tiles_n = (int)t32n;
      a.ntiles = (int)(t32m * t32n);
      void *args[] = {&a};
      const void *fn = akc ? (bkc ? small_kernel_for<true, true>(k) : small_kernel_for<true, false>(k))
                           : (bkc ? small_kernel_for<false, true>(k) : small_kernel_for<false, false>(k));
      WGB_CHECK_HIP(hipLaunchKernel(fn, dim3((unsigned)a.ntiles), dim3(64 * kSmallWaves), args, 0,
                                    ctx->stream));
      WGB_CHECK_LAUNCH("gemm_small_kernel");
      return WGB_OK;
    }
  }
  // VEC: the path that copies k-tiles straight into LDS with 32-bit lane
  // offsets from the tile origin, which stay below 256 * ld * sizeof(T) (a
  // tile spans at most 128 rows or k-rows of ld elements); larger leading
  // dimensions take the register path (same results, same loads). It takes
  // 16-byte aligned operand vectors, and fp32 operands that are only
  // element-aligned (ld not a multiple of 4 or a misaligned base: each
  // 16-byte copy then reads four dword-aligned floats, which CDNA's loads
  // allow), except NN, whose register path (B staged first) measured
  // faster there: on config 3's ragged 8191 x 8193 x 4097 (ld = 1 mod 64)
  // the copies took NT / TN / TT from 4037 / 4015 / 4055 to 3897 / 3879 /
  // 3895 us per launch and NN from 3992 to 4082.
  const int64_t off_cap = (int64_t)1 << 31;
  const bool offs32 = 256 * lda * (int64_t)sizeof(T) < off_cap && 256 * ldb * (int64_t)sizeof(T) < off_cap;
  const bool aligned = (lda % VW == 0) && (ldb % VW == 0) && aligned16(A) && aligned16(B);
  const bool vec = offs32 && (aligned || (sizeof(T) == 4 && (akc || !bkc)));
  if constexpr (sizeof(T) == 4) {
    // Wide tier: whole 256 x 128 tiles filling whole rounds of two blocks
    // per CU over a long k (8192^3: 2048 tiles, four rounds), 16-byte
    // aligned operands and full C only;
    // everything else (edge tiles, triangles, bands, split-k tails, the
    // two-part k range) stays on the 128 / 64 tiers.
    const int64_t wtiles = (m / kWideM) * (n / kWideN);
    if (vec && aligned && c_aligned && uplo == 0 && band == wgb::kBandNone && !A2 && m % kWideM == 0 &&
        n % kWideN == 0 && k % kWideBK == 0 && k >= 1024 && wtiles > 0 && wtiles % (2 * fill) == 0 &&
        wtiles <= INT32_MAX) {
      a.tiles_m = (int)(m / kWideM);
      a.tiles_n = (int)(n / kWideN);
      a.ntiles = (int)wtiles;
      a.nregular = a.ntiles;
      a.splits = 1;
      a.kt_split = (int)(k / kWideBK);
      a.ws = nullptr;
      void *args[] = {&a};
      const void *fn = akc ? (bkc ? reinterpret_cast<const void *>(gemm_wide_kernel<true, true>)
                                  : reinterpret_cast<const void *>(gemm_wide_kernel<true, false>))
                           : (bkc ? reinterpret_cast<const void *>(gemm_wide_kernel<false, true>)
                                  : reinterpret_cast<const void *>(gemm_wide_kernel<false, false>));
      WGB_CHECK_HIP(hipLaunchKernel(fn, dim3((unsigned)wtiles), dim3(kThreads), args, 0, ctx->stream));
      WGB_CHECK_LAUNCH("gemm_wide_kernel");
      return WGB_OK;
    }
  }
  if (A2) {
    constexpr int BK = 128 / (int)sizeof(T);
    if (!(vec && aligned && aligned16(A2) && aligned16(B2) && k % BK == 0 && akc == bkc &&
          band == wgb::kBandNone)) {
      int st = gemm_launch<T>(ctx, uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                              band, wsrc);
      if (st) return st;
      return gemm_launch<T>(ctx, uplo, transA, transB, m, n, k, alpha, A2, lda, B2, ldb, (T)1, C, ldc,
                            band, wsrc);
    }
    if (2 * k > INT32_MAX) return wgb::fail(WGB_ERR_INVALID_VALUE, "k too large for one two-part launch");
    a.k = 2 * k;
    a.A2 = A2;
    a.B2 = B2;
    a.kt_switch = (int)(k / BK);
  }
  auto count = [&](int64_t bt, int64_t &tmn, int64_t &tnn) {
    tmn = (m + bt - 1) / bt;
    tnn = (n + bt - 1) / bt;
    if (uplo == WGB_LOWER) return triangle_tiles(tmn, tnn);
    if (uplo == WGB_UPPER) return triangle_tiles(tnn, tmn);
    return tmn * tnn;
  };
  // 128-tiles once they fill whole rounds of two blocks per CU, or exactly
  // one block per CU over a long k; otherwise 64-tiles, whose rounds of
  // about four blocks per CU leave fewer CUs idle or half loaded. Measured
  // (TFLOP/s, 128 -> 64 tier): 2048 x 3072 x 4096 (384 tiles) 109.5 -> 126.0,
  // 1024 x 4096 x 1024 (256) 114.0 -> 119.0, 512 x 8192 x 512 (256) 94.3 ->
  // 102.6, 2048 x 2048 x 2048 (256) 128.5 -> 129.6; 2048 x 2048 x 8192 (256)
  // 141.0 -> 138.9 stays on 128-tiles.
  int64_t tm128, tn128;
  int64_t tiles128 = count(128, tm128, tn128);
  const int bt = (tiles128 >= 2 * fill || (tiles128 == fill && k >= 4096)) ? 128 : 64;
  int64_t tmn, tnn;
  int64_t ntiles = count(bt, tmn, tnn);
  if (ntiles > INT32_MAX) return wgb::fail(WGB_ERR_INVALID_VALUE, "problem too large for one launch");
  a.tiles_m = (int)tmn;
  a.tiles_n = (int)tnn;
  a.ntiles = (int)ntiles;
  int st = bt == 128 ? launch_tier<T, 128>(ctx, a, akc, bkc, vec, wsrc)
                     : launch_tier<T, 64>(ctx, a, akc, bkc, vec, wsrc);
  if (st) return st;
  WGB_CHECK_LAUNCH("gemm_kernel");
  return WGB_OK;
}

template <typename T>
int gemm_run(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t m, int64_t n, int64_t k,
             T alpha, const T *A, int64_t lda, const T *B, int64_t ldb, T beta, T *C,
             int64_t ldc, WsSource wsrc = WsSource()) {
  if (m == 0 || n == 0) return WGB_OK;
  wgb::timing_begin(ctx);
  int st = gemm_launch<T>(ctx, uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                          wgb::kBandNone, wsrc);
  if (st) return st;
  wgb::timing_end(ctx);
  return WGB_OK;
}

}  // namespace

namespace wgb {

int gemm_f32(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t m, int64_t n, int64_t k,
             float alpha, const float *A, int64_t lda, const float *B, int64_t ldb, float beta,
             float *C, int64_t ldc, int band) {
  return gemm_launch<float>(ctx, uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                            band);
}

int gemm_f64(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t m, int64_t n, int64_t k,
             double alpha, const double *A, int64_t lda, const double *B, int64_t ldb,
             double beta, double *C, int64_t ldc, int band) {
  return gemm_launch<double>(ctx, uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C,
                             ldc, band);
}

int gemm_side_f32(wgb_ctx *ctx, int transA, int transB, int64_t m, int64_t n, int64_t k, float alpha,
                  const float *A, int64_t lda, const float *B, int64_t ldb, float *C, int64_t ldc,
                  int band, const float *side) {
  return gemm_launch<float>(ctx, 0, transA, transB, m, n, k, alpha, A, lda, B, ldb, 0.f, C, ldc, band,
                            WsSource(), nullptr, nullptr, side);
}

int gemm_side_f64(wgb_ctx *ctx, int transA, int transB, int64_t m, int64_t n, int64_t k, double alpha,
                  const double *A, int64_t lda, const double *B, int64_t ldb, double *C, int64_t ldc,
                  int band, const double *side) {
  return gemm_launch<double>(ctx, 0, transA, transB, m, n, k, alpha, A, lda, B, ldb, 0.0, C, ldc, band,
                             WsSource(), nullptr, nullptr, side);
}

int gemm2_f32(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t m, int64_t n, int64_t k,
              float alpha, const float *A, const float *A2, int64_t lda, const float *B,
              const float *B2, int64_t ldb, float beta, float *C, int64_t ldc) {
  return gemm_launch<float>(ctx, uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                            wgb::kBandNone, WsSource(), A2, B2);
}

int gemm2_f64(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t m, int64_t n, int64_t k,
              double alpha, const double *A, const double *A2, int64_t lda, const double *B,
              const double *B2, int64_t ldb, double beta, double *C, int64_t ldc) {
  return gemm_launch<double>(ctx, uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                             wgb::kBandNone, WsSource(), A2, B2);
}

int check_gemm(int uplo, bool want_uplo, int transA, int transB, int64_t m, int64_t n, int64_t k,
               const void *A, int64_t lda, const void *B, int64_t ldb, const void *C,
               int64_t ldc) {
  return check_gemm_args(uplo, want_uplo, transA, transB, m, n, k, A, lda, B, ldb, C, ldc);
}

}  // namespace wgb

extern "C" int wgb_sgemm(wgb_ctx *ctx, int transA, int transB, int64_t m, int64_t n, int64_t k,
                         float alpha, const float *A, int64_t lda, const float *B, int64_t ldb,
                         float beta, float *C, int64_t ldc) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_gemm_args(0, false, transA, transB, m, n, k, A, lda, B, ldb, C, ldc))) return st;
  return gemm_run<float>(ctx, 0, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc);
}

// wgb_sgemm's launches with the split-k partials in the library's fixed
// per-GPU array (noalloc.hip): no hipMalloc, hipFree or other allocation on
// this path. Calls that overlap on one GPU share the array.
extern "C" int wgb_sgemm_noalloc(wgb_ctx *ctx, int transA, int transB, int64_t m, int64_t n,
                                 int64_t k, float alpha, const float *A, int64_t lda,
                                 const float *B, int64_t ldb, float beta, float *C, int64_t ldc) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_gemm_args(0, false, transA, transB, m, n, k, A, lda, B, ldb, C, ldc))) return st;
  WsSource ws;
  if ((st = wgb::noalloc_workspace(ctx, &ws.ptr))) return st;
  ws.bytes = wgb::kNoallocWsBytes;
  return gemm_run<float>(ctx, 0, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, ws);
}

extern "C" int wgb_sgemmtr(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t m, int64_t n,
                           int64_t k, float alpha, const float *A, int64_t lda, const float *B,
                           int64_t ldb, float beta, float *C, int64_t ldc) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_gemm_args(uplo, true, transA, transB, m, n, k, A, lda, B, ldb, C, ldc))) return st;
  return gemm_run<float>(ctx, uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc);
}

extern "C" int wgb_ssyrk(wgb_ctx *ctx, int uplo, int trans, int64_t n, int64_t k, float alpha,
                         const float *A, int64_t lda, float beta, float *C, int64_t ldc) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if (trans != WGB_NO_TRANS && trans != WGB_TRANS)
    return wgb::fail(WGB_ERR_INVALID_VALUE, "trans must be WGB_NO_TRANS or WGB_TRANS");
  // C = alpha*op(A)*op(A)^T + beta*C is sgemmtr with B = A and the opposite
  // trans flag: no copy of A is made.
  const int transB = trans == WGB_NO_TRANS ? WGB_TRANS : WGB_NO_TRANS;
  if ((st = check_gemm_args(uplo, true, trans, transB, n, n, k, A, lda, A, lda, C, ldc))) return st;
  return gemm_run<float>(ctx, uplo, trans, transB, n, n, k, alpha, A, lda, A, lda, beta, C, ldc);
}

extern "C" int wgb_dgemm(wgb_ctx *ctx, int transA, int transB, int64_t m, int64_t n, int64_t k,
                         double alpha, const double *A, int64_t lda, const double *B, int64_t ldb,
                         double beta, double *C, int64_t ldc) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_gemm_args(0, false, transA, transB, m, n, k, A, lda, B, ldb, C, ldc))) return st;
  // Reference BLAS quick return kept by wgblas (src/dgemm/dgemm.mjs:177-179).
  if ((alpha == 0.0 || k == 0) && beta == 1.0) return WGB_OK;
  return gemm_run<double>(ctx, 0, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc);
}

extern "C" int wgb_dgemmtr(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t m, int64_t n,
                           int64_t k, double alpha, const double *A, int64_t lda, const double *B,
                           int64_t ldb, double beta, double *C, int64_t ldc) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_gemm_args(uplo, true, transA, transB, m, n, k, A, lda, B, ldb, C, ldc))) return st;
  // dgemm's quick return (src/dgemmtr/dgemmtr.mjs:189).
  if ((alpha == 0.0 || k == 0) && beta == 1.0) return WGB_OK;
  return gemm_run<double>(ctx, uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc);
}

extern "C" int wgb_dsyrk(wgb_ctx *ctx, int uplo, int trans, int64_t n, int64_t k, double alpha,
                         const double *A, int64_t lda, double beta, double *C, int64_t ldc) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if (trans != WGB_NO_TRANS && trans != WGB_TRANS)
    return wgb::fail(WGB_ERR_INVALID_VALUE, "trans must be WGB_NO_TRANS or WGB_TRANS");
  const int transB = trans == WGB_NO_TRANS ? WGB_TRANS : WGB_NO_TRANS;
  if ((st = check_gemm_args(uplo, true, trans, transB, n, n, k, A, lda, A, lda, C, ldc))) return st;
  // dgemm's quick return (src/dsyrk/dsyrk.mjs:142).
  if ((alpha == 0.0 || k == 0) && beta == 1.0) return WGB_OK;
  return gemm_run<double>(ctx, uplo, trans, transB, n, n, k, alpha, A, lda, A, lda, beta, C, ldc);
}
