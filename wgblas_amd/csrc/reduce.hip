// Level-1 reductions: sdot, sasum, snrm2, isamax and their native-fp64
// counterparts ddot, dasum, dnrm2, idamax.
//
// wgblas runs each of these as two compute passes on one encoder: 128
// workgroups of 64 threads grid-stride over x with four accumulators each,
// then a single workgroup folds the 128 partials (src/sdot/sdot.mjs:86-92,
// src/shaders/sdot.wgsl, src/shaders/reduction/sum.wgsl). This file keeps the
// two-stage structure and its determinism, sized for MI355X's HBM:
//
//  * stage 1 uses G = min(4096, ceil(n / 4096)) blocks of 256 threads, each
//    reading one contiguous range of x (and y); G and the ranges depend only
//    on n, so the summation order (and the result) is the same on every run
//    and every device;
//  * unit-stride, 16-byte-aligned operands are read with 16-byte
//    non-temporal loads, sixteen in flight per lane per input; strides 2..4
//    read their span the same way and keep every incx-th element; other
//    strides read one element per lane;
//  * a block folds its lanes with 64-lane shuffles, then its four waves in
//    LDS, in a fixed order, and stores one partial;
//  * stage 2 (one block, a second launch) folds the G partials in a fixed
//    order and applies the final combine (snrm2) or index pick (isamax).
//
// The per-element arithmetic follows the WGSL kernels: f32 accumulation,
// snrm2's big/medium/small classification with the same power-of-two
// thresholds and scales (src/shaders/snrm2.wgsl:33-51), LAPACK 3.10's combine
// (src/shaders/reduction/scaledSum.wgsl:50-101), and isamax's strict '>'
// with a -1 sentinel and lower-index tie break (src/shaders/isamax.wgsl:28-80,
// src/shaders/reduction/argmax.wgsl). The fp64 routines (wgblas emulates
// them in double-double: src/shaders/{ddot,dasum,dnrm2,idamax}.wgsl,
// reduction/*F64.wgsl) accumulate in native f64 with the same rules; dnrm2
// uses Blue's algorithm with LAPACK 3.10's dnrm2 thresholds for IEEE double
// (wgblas moves them to fit double-double's f32 exponent range).
#include "common.h"

#include <type_traits>

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef double v2d __attribute__((ext_vector_type(2)));
typedef double v4d __attribute__((ext_vector_type(4)));

// The 16-byte vector of an element type: W elements.
template <typename T>
struct Vec16;
template <>
struct Vec16<float> {
  typedef v4f type;
  static constexpr int W = 4;
};
template <>
struct Vec16<double> {
  typedef v2d type;
  static constexpr int W = 2;
};

constexpr int kThreads = 256;
// 16-byte loads in flight per lane and input, and (common.h) at most 4096
// first-pass blocks: measured at 2^28 on MI355X against 8 loads / 2048
// blocks, +1-2.5% (sdot 6.97, sasum 6.86, snrm2 6.86, isamax 6.81 TB/s;
// the box's read roof measured by roof_probe: 7.1 TB/s).
constexpr int kUnroll = 16;
constexpr int64_t kElemsPerBlockMin = 4096;

// snrm2 thresholds and scales (powers of two): src/shaders/snrm2.wgsl:33-36.
constexpr float kTsml = 0x1p-63f;
constexpr float kTbig = 0x1p50f;
constexpr float kSsml = 0x1p75f;
constexpr float kSbig = 0x1p-76f;
constexpr int kSbigSqExp = -152;  // log2(SBIG^2)

// dnrm2 thresholds and scales for IEEE double, LAPACK 3.10's dnrm2
// (la_constants: tsml = 2^ceil((minexp-1)/2), tbig = 2^floor((maxexp-digits+1)/2),
// ssml = 2^-floor((minexp-digits)/2), sbig = 2^-ceil((maxexp+digits-1)/2)).
constexpr double kDTsml = 0x1p-511;
constexpr double kDTbig = 0x1p486;
constexpr double kDSsml = 0x1p537;
constexpr double kDSbig = 0x1p-538;

// Partial slots in the context scratch (the largest Partial is dnrm2's).
constexpr size_t kPartialBytes = 32;

int reduce_blocks(int64_t n) {
  int64_t g = (n + kElemsPerBlockMin - 1) / kElemsPerBlockMin;
  if (g > wgb::kMaxReduceBlocks) g = wgb::kMaxReduceBlocks;
  if (g < 1) g = 1;
  return (int)g;
}

using wgb::aligned16;

// ---- the four reductions as accumulate / merge policies -------------------
//
// State: what one lane accumulates. Partial: what a block (and pass 2)
// merges. addv takes one 16-byte vector (W consecutive elements starting at
// element index `i`); add1 takes one element, `c` naming an accumulation
// chain the policy may use for ILP (taken modulo its chain count).

__device__ __forceinline__ v4f nt_load(const v4f *p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ v2d nt_load(const v2d *p) { return __builtin_nontemporal_load(p); }

struct SdotOp {
  typedef float Elem;
  typedef v4f V;
  static constexpr int NIN = 2;
  typedef v4f State;
  typedef float Partial;
  __device__ static State init() { return v4f{0.f, 0.f, 0.f, 0.f}; }
  __device__ static void addv(State &s, v4f a, v4f b, int64_t) {
    s.x = fmaf(a.x, b.x, s.x);
    s.y = fmaf(a.y, b.y, s.y);
    s.z = fmaf(a.z, b.z, s.z);
    s.w = fmaf(a.w, b.w, s.w);
  }
  __device__ static void add1(State &s, float a, float b, int64_t, int c) { s[c] = fmaf(a, b, s[c]); }
  __device__ static Partial finish(State s) { return (s.x + s.y) + (s.z + s.w); }
  __device__ static Partial identity() { return 0.0f; }
  __device__ static Partial merge(Partial a, Partial b) { return a + b; }
  __device__ static Partial shfl(Partial a, int off) { return __shfl_xor(a, off, 64); }
  typedef float Result;
  __device__ static Result result(Partial p) { return p; }
};

struct SasumOp {
  typedef float Elem;
  typedef v4f V;
  static constexpr int NIN = 1;
  typedef v4f State;
  typedef float Partial;
  __device__ static State init() { return v4f{0.f, 0.f, 0.f, 0.f}; }
  __device__ static void addv(State &s, v4f a, v4f, int64_t) {
    s.x += fabsf(a.x);
    s.y += fabsf(a.y);
    s.z += fabsf(a.z);
    s.w += fabsf(a.w);
  }
  __device__ static void add1(State &s, float a, float, int64_t, int c) { s[c] += fabsf(a); }
  __device__ static Partial finish(State s) { return (s.x + s.y) + (s.z + s.w); }
  __device__ static Partial identity() { return 0.0f; }
  __device__ static Partial merge(Partial a, Partial b) { return a + b; }
  __device__ static Partial shfl(Partial a, int off) { return __shfl_xor(a, off, 64); }
  typedef float Result;
  __device__ static Result result(Partial p) { return p; }
};

// snrm2: (big, medium, small) sums of scaled squares.
struct Nrm {
  float big, med, sml;
};

// Adds |v|'s contribution as snrm2.wgsl's accum() does: NaN fails both
// tests and lands in medium, which the combine turns into a NaN result.
__device__ __forceinline__ void nrm_accum(Nrm &s, float v) {
  float ax = fabsf(v);
  bool big = ax > kTbig;
  bool sml = ax < kTsml;
  float yb = ax * kSbig;
  float ys = ax * kSsml;
  s.big = big ? fmaf(yb, yb, s.big) : s.big;
  s.med = (big || sml) ? s.med : fmaf(ax, ax, s.med);
  s.sml = sml ? fmaf(ys, ys, s.sml) : s.sml;
}

struct Snrm2Op {
  typedef float Elem;
  typedef v4f V;
  static constexpr int NIN = 1;
  typedef Nrm State;
  typedef v4f Partial;  // (big, medium, small, 0)
  __device__ static State init() { return Nrm{0.f, 0.f, 0.f}; }
  __device__ static void addv(State &s, v4f a, v4f, int64_t) {
    // Whole-wave fast path: when every lane's four |x| lie in
    // [TSML, TBIG], the squares go straight into the medium sum. (min/max
    // skip NaN, which then takes the fast path into the medium sum, exactly
    // where the classification puts it.)
    const float hi = fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w)));
    const float lo = fminf(fminf(fabsf(a.x), fabsf(a.y)), fminf(fabsf(a.z), fabsf(a.w)));
    const bool odd = !(hi <= kTbig) || lo < kTsml;
    if (__any(odd)) {
      nrm_accum(s, a.x);
      nrm_accum(s, a.y);
      nrm_accum(s, a.z);
      nrm_accum(s, a.w);
    } else {
      s.med = fmaf(a.x, a.x, s.med);
      s.med = fmaf(a.y, a.y, s.med);
      s.med = fmaf(a.z, a.z, s.med);
      s.med = fmaf(a.w, a.w, s.med);
    }
  }
  __device__ static void add1(State &s, float a, float, int64_t, int) { nrm_accum(s, a); }
  // The elements of a whose bit is set in `keep` (reduce_span's every
  // INC-th element), in order, with addv's whole-wave fast path; the other
  // elements are left out of the test and of the sums.
  __device__ static void add_kept(State &s, v4f a, uint32_t keep) {
    float hi = 0.f, lo = 1.f;  // 1: a medium value, neutral for the test
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float ax = fabsf(a[c]);
      const bool k = (keep >> c) & 1u;
      hi = k ? fmaxf(hi, ax) : hi;
      lo = k ? fminf(lo, ax) : lo;
    }
    const bool odd = !(hi <= kTbig) || lo < kTsml;
    if (__any(odd)) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if ((keep >> c) & 1u) nrm_accum(s, a[c]);
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) s.med = ((keep >> c) & 1u) ? fmaf(a[c], a[c], s.med) : s.med;
    }
  }
  __device__ static Partial finish(State s) { return v4f{s.big, s.med, s.sml, 0.f}; }
  __device__ static Partial identity() { return v4f{0.f, 0.f, 0.f, 0.f}; }
  __device__ static Partial merge(Partial a, Partial b) { return a + b; }
  __device__ static Partial shfl(Partial a, int off) {
    return v4f{__shfl_xor(a.x, off, 64), __shfl_xor(a.y, off, 64), __shfl_xor(a.z, off, 64), 0.f};
  }
  typedef float Result;
  __device__ static Result result(Partial p);  // LAPACK combine, defined below
};

// isamax: (max |x|, its first index). A lane visits its elements in
// increasing index order, so the strict '>' keeps the first occurrence;
// merges prefer the larger value, then the lower index. The -1 sentinel
// loses to every |x| >= 0, and NaN never compares greater, so it is skipped.
struct AmaxPartial {
  float val;
  float pad;
  int64_t idx;
};

__device__ __forceinline__ void amax_step(AmaxPartial &s, float v, int64_t i) {
  float ax = fabsf(v);
  if (ax > s.val) {
    s.val = ax;
    s.idx = i;
  }
}

struct IsamaxOp {
  typedef float Elem;
  typedef v4f V;
  static constexpr int NIN = 1;
  typedef AmaxPartial State;
  typedef AmaxPartial Partial;
  __device__ static State init() { return AmaxPartial{-1.0f, 0.f, 0}; }
  __device__ static void addv(State &s, v4f a, v4f, int64_t i) {
    // max|x| of the four first (v_max ignores a NaN operand, so NaN never
    // wins); only a vector that beats the running best is searched, for
    // its first element equal to that max.
    const float m = fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w)));
    if (m > s.val) {
      const int c = fabsf(a.x) == m ? 0 : fabsf(a.y) == m ? 1 : fabsf(a.z) == m ? 2 : 3;
      s.val = m;
      s.idx = i + c;
    }
  }
  __device__ static void add1(State &s, float a, float, int64_t i, int) { amax_step(s, a, i); }
  __device__ static Partial finish(State s) { return s; }
  __device__ static Partial identity() { return AmaxPartial{-1.0f, 0.f, 0}; }
  __device__ static Partial merge(Partial a, Partial b) {
    return (b.val > a.val || (b.val == a.val && b.idx < a.idx)) ? b : a;
  }
  __device__ static Partial shfl(Partial a, int off) {
    return AmaxPartial{__shfl_xor(a.val, off, 64), 0.f, __shfl_xor(a.idx, off, 64)};
  }
  typedef int64_t Result;
  __device__ static Result result(Partial p) { return p.idx; }
};

// ---- fp64 policies ---------------------------------------------------------

struct DdotOp {
  typedef double Elem;
  typedef v2d V;
  static constexpr int NIN = 2;
  typedef v2d State;
  typedef double Partial;
  __device__ static State init() { return v2d{0.0, 0.0}; }
  __device__ static void addv(State &s, v2d a, v2d b, int64_t) {
    s.x = fma(a.x, b.x, s.x);
    s.y = fma(a.y, b.y, s.y);
  }
  __device__ static void add1(State &s, double a, double b, int64_t, int c) {
    s[c & 1] = fma(a, b, s[c & 1]);
  }
  __device__ static Partial finish(State s) { return s.x + s.y; }
  __device__ static Partial identity() { return 0.0; }
  __device__ static Partial merge(Partial a, Partial b) { return a + b; }
  __device__ static Partial shfl(Partial a, int off) { return __shfl_xor(a, off, 64); }
  typedef double Result;
  __device__ static Result result(Partial p) { return p; }
};

struct DasumOp {
  typedef double Elem;
  typedef v2d V;
  static constexpr int NIN = 1;
  typedef v2d State;
  typedef double Partial;
  __device__ static State init() { return v2d{0.0, 0.0}; }
  __device__ static void addv(State &s, v2d a, v2d, int64_t) {
    s.x += fabs(a.x);
    s.y += fabs(a.y);
  }
  __device__ static void add1(State &s, double a, double, int64_t, int c) { s[c & 1] += fabs(a); }
  __device__ static Partial finish(State s) { return s.x + s.y; }
  __device__ static Partial identity() { return 0.0; }
  __device__ static Partial merge(Partial a, Partial b) { return a + b; }
  __device__ static Partial shfl(Partial a, int off) { return __shfl_xor(a, off, 64); }
  typedef double Result;
  __device__ static Result result(Partial p) { return p; }
};

struct NrmD {
  double big, med, sml;
};

// dnrm2's classification, as nrm_accum with LAPACK's double constants: NaN
// fails both tests and lands in medium; Inf lands in big.
__device__ __forceinline__ void nrmd_accum(NrmD &s, double v) {
  double ax = fabs(v);
  bool big = ax > kDTbig;
  bool sml = ax < kDTsml;
  double yb = ax * kDSbig;
  double ys = ax * kDSsml;
  s.big = big ? fma(yb, yb, s.big) : s.big;
  s.med = (big || sml) ? s.med : fma(ax, ax, s.med);
  s.sml = sml ? fma(ys, ys, s.sml) : s.sml;
}

struct Dnrm2Op {
  typedef double Elem;
  typedef v2d V;
  static constexpr int NIN = 1;
  typedef NrmD State;
  typedef v4d Partial;  // (big, medium, small, 0)
  __device__ static State init() { return NrmD{0.0, 0.0, 0.0}; }
  __device__ static void addv(State &s, v2d a, v2d, int64_t) {
    // Whole-wave fast path as in snrm2 (min/max skip NaN, which then goes
    // to the medium sum, where the classification puts it).
    const double hi = fmax(fabs(a.x), fabs(a.y));
    const double lo = fmin(fabs(a.x), fabs(a.y));
    const bool odd = !(hi <= kDTbig) || lo < kDTsml;
    if (__any(odd)) {
      nrmd_accum(s, a.x);
      nrmd_accum(s, a.y);
    } else {
      s.med = fma(a.x, a.x, s.med);
      s.med = fma(a.y, a.y, s.med);
    }
  }
  __device__ static void add1(State &s, double a, double, int64_t, int) { nrmd_accum(s, a); }
  __device__ static Partial finish(State s) { return v4d{s.big, s.med, s.sml, 0.0}; }
  __device__ static Partial identity() { return v4d{0.0, 0.0, 0.0, 0.0}; }
  __device__ static Partial merge(Partial a, Partial b) { return a + b; }
  __device__ static Partial shfl(Partial a, int off) {
    return v4d{__shfl_xor(a.x, off, 64), __shfl_xor(a.y, off, 64), __shfl_xor(a.z, off, 64), 0.0};
  }
  typedef double Result;
  __device__ static Result result(Partial p);  // LAPACK combine, defined below
};

struct AmaxPartialD {
  double val;
  int64_t idx;
};

// idamax: isamax's rules on doubles (strict '>', -1 sentinel, NaN never
// selected, lower index on ties).
struct IdamaxOp {
  typedef double Elem;
  typedef v2d V;
  static constexpr int NIN = 1;
  typedef AmaxPartialD State;
  typedef AmaxPartialD Partial;
  __device__ static State init() { return AmaxPartialD{-1.0, 0}; }
  __device__ static void addv(State &s, v2d a, v2d, int64_t i) {
    const double m = fmax(fabs(a.x), fabs(a.y));
    if (m > s.val) {
      s.idx = i + (fabs(a.x) == m ? 0 : 1);
      s.val = m;
    }
  }
  __device__ static void add1(State &s, double a, double, int64_t i, int) {
    const double ax = fabs(a);
    if (ax > s.val) {
      s.val = ax;
      s.idx = i;
    }
  }
  __device__ static Partial finish(State s) { return s; }
  __device__ static Partial identity() { return AmaxPartialD{-1.0, 0}; }
  __device__ static Partial merge(Partial a, Partial b) {
    return (b.val > a.val || (b.val == a.val && b.idx < a.idx)) ? b : a;
  }
  __device__ static Partial shfl(Partial a, int off) {
    return AmaxPartialD{__shfl_xor(a.val, off, 64), __shfl_xor(a.idx, off, 64)};
  }
  typedef int64_t Result;
  __device__ static Result result(Partial p) { return p.idx; }
};

// ---- block merge (fixed order) --------------------------------------------

template <class Op>
__device__ __forceinline__ typename Op::Partial block_merge(typename Op::Partial p) {
  __shared__ typename Op::Partial lds[kThreads / 64];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) p = Op::merge(p, Op::shfl(p, off));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) lds[wave] = p;
  __syncthreads();
  if (threadIdx.x == 0) {
    p = Op::merge(Op::merge(lds[0], lds[1]), Op::merge(lds[2], lds[3]));
  }
  return p;
}

// Block b's share of [0, total) units: one contiguous range, its start a
// multiple of 8 units, depending only on total and the grid size. Reading
// whole contiguous ranges per block streams HBM better than a grid-stride
// walk (measured on MI355X: ~7.0 vs ~5.5 TB/s for a read-only pass).
__device__ __forceinline__ void chunk_of(int64_t total, int64_t &beg, int64_t &end) {
  int64_t per = (total + gridDim.x - 1) / gridDim.x;
  per = (per + 7) & ~(int64_t)7;
  beg = per * blockIdx.x;
  end = beg + per < total ? beg + per : total;
  if (beg > end) beg = end;
}

// A block's partial goes to its slot; stage 2 (fold_kernel) folds them.
// (Folding in the last block of the same launch needs an agent-scope
// release per block, which writes back the XCD's L2: measured ~90 us per
// 2048-block launch on MI355X, far more than the second launch costs.)
template <class Op>
__device__ __forceinline__ void finish(typename Op::Partial p, typename Op::Partial *partials) {
  if (threadIdx.x == 0) partials[blockIdx.x] = p;
}

// Unit-stride, 16-byte-aligned operands: 16-byte non-temporal loads,
// kUnroll of them in flight per lane per input.
template <class Op>
__global__ __launch_bounds__(kThreads) void reduce_vec(const typename Op::Elem *__restrict__ x,
                                                       const typename Op::Elem *__restrict__ y, int64_t n,
                                                       typename Op::Partial *__restrict__ partials) {
  typedef typename Op::V V;
  constexpr int W = Vec16<typename Op::Elem>::W;
  const V *xv = reinterpret_cast<const V *>(x);
  const V *yv = reinterpret_cast<const V *>(y);
  const int64_t nv = n / W;
  int64_t beg, end;
  chunk_of(nv, beg, end);
  typename Op::State s = Op::init();
  int64_t q = beg + threadIdx.x;
  for (; q + (kUnroll - 1) * kThreads < end; q += kUnroll * kThreads) {
    V a[kUnroll], b[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      a[u] = nt_load(xv + q + u * kThreads);
      b[u] = Op::NIN == 2 ? nt_load(yv + q + u * kThreads) : a[u];
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) Op::addv(s, a[u], b[u], W * (q + u * kThreads));
  }
  for (; q < end; q += kThreads) {
    V a = xv[q];
    Op::addv(s, a, Op::NIN == 2 ? yv[q] : a, W * q);
  }
  // The n % W trailing elements follow the last block's range.
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0)
    for (int64_t i = nv * W; i < n; ++i)
      Op::add1(s, x[i], Op::NIN == 2 ? y[i] : (typename Op::Elem)0, i, 0);
  finish<Op>(block_merge<Op>(Op::finish(s)), partials);
}

// Whether Op has add_kept (a vector of which some elements are kept).
template <class Op, class = void>
struct HasKept : std::false_type {};
template <class Op>
struct HasKept<Op, std::void_t<decltype(&Op::add_kept)>> : std::true_type {};

// Which of the W elements of 16-byte vector v of the span are kept (every
// INC-th element): a pattern that repeats every INC vectors (W = 4) or
// INC / gcd vectors (W = 2), looked up from v mod INC.
template <int W, int INC>
__device__ __forceinline__ uint32_t kept_mask(uint32_t v) {
  const uint32_t r = v % INC;
  uint32_t keep = 0u;
#pragma unroll
  for (int c = 0; c < W; ++c) {
    // element W v + c is kept iff (W r + c) % INC == 0 (W v = W r mod INC)
    uint32_t bit = 0u;
#pragma unroll
    for (int rr = 0; rr < INC; ++rr) bit |= (r == (uint32_t)rr && (W * rr + c) % INC == 0) ? 1u : 0u;
    keep |= bit << c;
  }
  return keep;
}

// Small constant strides (incx == incy == INC, 2..4): read the whole span
// [0, (n-1)*INC] with the same coalesced 16-byte loads and keep every
// INC-th element. The span's lines are fetched either way, so this trades
// nothing in HBM bytes for far fewer, wider load instructions.
template <class Op, int INC>
__global__ __launch_bounds__(kThreads) void reduce_span(const typename Op::Elem *__restrict__ x,
                                                        const typename Op::Elem *__restrict__ y, int64_t n,
                                                        typename Op::Partial *__restrict__ partials) {
  typedef typename Op::V V;
  constexpr int W = Vec16<typename Op::Elem>::W;
  const V *xv = reinterpret_cast<const V *>(x);
  const V *yv = reinterpret_cast<const V *>(y);
  const uint32_t span = (uint32_t)((n - 1) * INC + 1);  // host checks span < 2^31
  const int64_t nv = span / W;
  int64_t beg, end;
  chunk_of(nv, beg, end);
  typename Op::State s = Op::init();
  uint32_t q = (uint32_t)(beg + threadIdx.x);
  for (; q + (kUnroll - 1) * kThreads < (uint32_t)end; q += kUnroll * kThreads) {
    V a[kUnroll], b[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      a[u] = nt_load(xv + q + u * kThreads);
      b[u] = Op::NIN == 2 ? nt_load(yv + q + u * kThreads) : a[u];
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if constexpr (HasKept<Op>::value) {
        Op::add_kept(s, a[u], kept_mask<W, INC>(q + u * kThreads));
      } else {
        // (the per-element test measured faster here for isamax, 0.82
        // against 0.80 of the span's HBM rate at incx 3, n = 2^26)
#pragma unroll
        for (int c = 0; c < W; ++c) {
          const uint32_t e = W * (q + u * kThreads) + c;
          if (e % INC == 0) Op::add1(s, a[u][c], b[u][c], e / INC, c);
        }
      }
    }
  }
  for (; q < (uint32_t)end; q += kThreads) {
    V a = xv[q];
    V b = Op::NIN == 2 ? yv[q] : a;
#pragma unroll
    for (int c = 0; c < W; ++c) {
      const uint32_t e = W * q + c;
      if (e % INC == 0) Op::add1(s, a[c], b[c], e / INC, c);
    }
  }
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0)
    for (uint32_t e = (uint32_t)nv * W; e < span; ++e)
      if (e % INC == 0) Op::add1(s, x[e], Op::NIN == 2 ? y[e] : (typename Op::Elem)0, e / INC, 0);
  finish<Op>(block_merge<Op>(Op::finish(s)), partials);
}

// Any positive strides (and misaligned unit stride): one element per lane
// per step, kUnroll steps in flight.
template <class Op>
__global__ __launch_bounds__(kThreads) void reduce_strided(const typename Op::Elem *__restrict__ x,
                                                           int64_t incx,
                                                           const typename Op::Elem *__restrict__ y,
                                                           int64_t incy, int64_t n,
                                                           typename Op::Partial *__restrict__ partials) {
  typedef typename Op::Elem T;
  int64_t beg, end;
  chunk_of(n, beg, end);
  typename Op::State s = Op::init();
  int64_t i = beg + threadIdx.x;
  for (; i + (kUnroll - 1) * kThreads < end; i += kUnroll * kThreads) {
    T a[kUnroll], b[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      a[u] = x[(i + u * kThreads) * incx];
      b[u] = Op::NIN == 2 ? y[(i + u * kThreads) * incy] : (T)0;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) Op::add1(s, a[u], b[u], i + u * kThreads, u & 3);
  }
  for (; i < end; i += kThreads) Op::add1(s, x[i * incx], Op::NIN == 2 ? y[i * incy] : (T)0, i, 0);
  finish<Op>(block_merge<Op>(Op::finish(s)), partials);
}

// Stage 2: one block folds the G partials in a fixed order (each thread
// issues all of its loads before folding them) and writes the result.
template <class Op>
__global__ __launch_bounds__(kThreads) void fold_kernel(const typename Op::Partial *__restrict__ partials,
                                                        int G, typename Op::Result *__restrict__ out) {
  constexpr int kPer = wgb::kMaxReduceBlocks / kThreads;
  typename Op::Partial v[kPer];
#pragma unroll
  for (int r = 0; r < kPer; ++r) {
    const int i = threadIdx.x + r * kThreads;
    v[r] = i < G ? partials[i] : Op::identity();
  }
  typename Op::Partial p = v[0];
#pragma unroll
  for (int r = 1; r < kPer; ++r) p = Op::merge(p, v[r]);
  p = block_merge<Op>(p);
  if (threadIdx.x == 0) *out = Op::result(p);
}

// v * 2^e by editing the exponent field, as scaledSum.wgsl's ldexpBits does:
// zero and results below the normal range give a signed 0, overflow a
// signed Inf, Inf and NaN pass through.
__device__ __forceinline__ float ldexp_bits(float v, int e) {
  uint32_t bits = __float_as_uint(v);
  uint32_t sign = bits & 0x80000000u;
  int ev = (int)((bits >> 23) & 0xffu);
  if (ev == 255) return v;
  int en = ev + e;
  if (ev == 0 || en <= 0) return __uint_as_float(sign);
  if (en >= 255) return __uint_as_float(sign | 0x7f800000u);
  return __uint_as_float((bits & 0x807fffffu) | ((uint32_t)en << 23));
}

__device__ __forceinline__ bool is_nan_bits(float v) {
  return (__float_as_uint(v) & 0x7fffffffu) > 0x7f800000u;
}

// LAPACK 3.10 combine of the three sums (scaledSum.wgsl:64-101).
__device__ float nrm_combine(float abig, float amed, float asml) {
  if (is_nan_bits(amed)) return amed;
  bool med_live = amed > 0.0f;
  float scl = 1.0f;
  float sumsq = amed;
  if (abig > 0.0f) {
    if (med_live) abig = abig + ldexp_bits(amed, kSbigSqExp);
    scl = 1.0f / kSbig;
    sumsq = abig;
  } else if (asml > 0.0f) {
    if (med_live) {
      amed = sqrtf(amed);
      asml = sqrtf(asml) / kSsml;
      float ymax = fmaxf(asml, amed);
      float ymin = fminf(asml, amed);
      float q = ymin / ymax;
      sumsq = ymax * ymax * (1.0f + q * q);
    } else {
      scl = 1.0f / kSsml;
      sumsq = asml;
    }
  }
  return scl * sqrtf(sumsq);
}

__device__ Snrm2Op::Result Snrm2Op::result(Partial p) { return nrm_combine(p.x, p.y, p.z); }

// LAPACK 3.10's dnrm2 combine of the three sums (a NaN medium sum gives NaN
// first, as snrm2's; an Inf lands in the big sum and gives Inf).
__device__ double nrmd_combine(double abig, double amed, double asml) {
  if (isnan(amed)) return amed;
  double scl = 1.0, sumsq = amed;
  if (abig > 0.0) {
    if (amed > 0.0) abig = abig + (amed * kDSbig) * kDSbig;
    scl = 1.0 / kDSbig;
    sumsq = abig;
  } else if (asml > 0.0) {
    if (amed > 0.0) {
      amed = sqrt(amed);
      asml = sqrt(asml) / kDSsml;
      double ymax = fmax(asml, amed), ymin = fmin(asml, amed);
      double q = ymin / ymax;
      sumsq = ymax * ymax * (1.0 + q * q);
    } else {
      scl = 1.0 / kDSsml;
      sumsq = asml;
    }
  }
  return scl * sqrt(sumsq);
}

__device__ Dnrm2Op::Result Dnrm2Op::result(Partial p) { return nrmd_combine(p.x, p.y, p.z); }

// Writes the n <= 0 answer of a `_dev` call with a kernel rather than a
// memset, so the call stays safe to capture in a HIP graph.
template <typename T>
__global__ void set_value(T *out, T v) {
  *out = v;
}

// ---- host side -------------------------------------------------------------

template <typename T>
int check_vec(int64_t n, const T *x, int64_t incx, const char *xname, const char *incname) {
  if (incx <= 0)
    return wgb::fail(WGB_ERR_INVALID_VALUE, std::string(incname) + " must be positive");
  if (n > 0 && !x) return wgb::fail(WGB_ERR_INVALID_VALUE, std::string(xname) + " is null");
  return WGB_OK;
}

void *partials_of(wgb_ctx *ctx) { return ctx->scratch; }
void *result_slot(wgb_ctx *ctx) {
  return (char *)ctx->scratch + (size_t)wgb::kMaxReduceBlocks * kPartialBytes;
}

// Stage 1 (the read pass) and stage 2 (the fold), two launches on the stream.
template <class Op>
int launch_reduce(wgb_ctx *ctx, int64_t n, const typename Op::Elem *x, int64_t incx,
                  const typename Op::Elem *y, int64_t incy, typename Op::Result *d_out,
                  const char *what) {
  static_assert(sizeof(typename Op::Partial) <= kPartialBytes, "partial slot too small");
  const int G = reduce_blocks(n);
  auto *part = (typename Op::Partial *)partials_of(ctx);
  int Gl = G;
  const bool same = Op::NIN == 1 || (incy == incx && aligned16(y));
  const int64_t span = (n - 1) * incx + 1;
  if (incx == 1 && aligned16(x) && same) {
    reduce_vec<Op><<<G, kThreads, 0, ctx->stream>>>(x, y, n, part);
  } else if (incx >= 2 && incx <= 4 && aligned16(x) && same && span < ((int64_t)1 << 31)) {
    // G from the span, not n: each block reads a span range.
    Gl = reduce_blocks(span);
    if (incx == 2)
      reduce_span<Op, 2><<<Gl, kThreads, 0, ctx->stream>>>(x, y, n, part);
    else if (incx == 3)
      reduce_span<Op, 3><<<Gl, kThreads, 0, ctx->stream>>>(x, y, n, part);
    else
      reduce_span<Op, 4><<<Gl, kThreads, 0, ctx->stream>>>(x, y, n, part);
  } else {
    reduce_strided<Op><<<G, kThreads, 0, ctx->stream>>>(x, incx, y, incy, n, part);
  }
  WGB_CHECK_LAUNCH(what);
  fold_kernel<Op><<<1, kThreads, 0, ctx->stream>>>(part, Gl, d_out);
  WGB_CHECK_LAUNCH(what);
  return WGB_OK;
}

// Copies a device scalar into the context's pinned slot and waits for it.
template <typename T>
int fetch_scalar(wgb_ctx *ctx, const T *d_src, T *host_dst) {
  WGB_CHECK_HIP(hipMemcpyAsync(ctx->host_result, d_src, sizeof(T), hipMemcpyDeviceToHost,
                               ctx->stream));
  WGB_CHECK_HIP(hipStreamSynchronize(ctx->stream));
  *host_dst = *(const T *)ctx->host_result;
  return WGB_OK;
}

// The `_dev` form: result written to device memory, n <= 0 gives `empty`
// (set by a kernel, so the call stays graph-capturable). y == nullptr for
// the one-vector routines.
template <class Op>
int reduce_to_device(wgb_ctx *ctx, int64_t n, const typename Op::Elem *x, int64_t incx,
                     const typename Op::Elem *y, int64_t incy, typename Op::Result *d_result,
                     typename Op::Result empty, const char *what) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_vec(n, x, incx, "x", "incx"))) return st;
  if (Op::NIN == 2 && (st = check_vec(n, y, incy, "y", "incy"))) return st;
  if (!d_result) return wgb::fail(WGB_ERR_INVALID_VALUE, "d_result is null");
  if (Op::NIN == 1) {
    y = x;
    incy = incx;
  }
  wgb::timing_begin(ctx);
  if (n <= 0)
    set_value<<<1, 1, 0, ctx->stream>>>(d_result, empty);
  else if ((st = launch_reduce<Op>(ctx, n, x, incx, y, incy, d_result, what)))
    return st;
  wgb::timing_end(ctx);
  return WGB_OK;
}

// The host-result form: n <= 0 returns `empty` without touching the device.
template <class Op>
int reduce_to_host(wgb_ctx *ctx, int64_t n, const typename Op::Elem *x, int64_t incx,
                   const typename Op::Elem *y, int64_t incy, typename Op::Result *result,
                   typename Op::Result empty, const char *what) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_vec(n, x, incx, "x", "incx"))) return st;
  if (Op::NIN == 2 && (st = check_vec(n, y, incy, "y", "incy"))) return st;
  if (!result) return wgb::fail(WGB_ERR_INVALID_VALUE, "result is null");
  if (n <= 0) {
    *result = empty;
    return WGB_OK;
  }
  if (Op::NIN == 1) {
    y = x;
    incy = incx;
  }
  auto *slot = (typename Op::Result *)result_slot(ctx);
  wgb::timing_begin(ctx);
  if ((st = launch_reduce<Op>(ctx, n, x, incx, y, incy, slot, what))) return st;
  wgb::timing_end(ctx);
  return fetch_scalar(ctx, slot, result);
}

}  // namespace

// ---- fp32 ---------------------------------------------------------------

extern "C" int wgb_sdot_dev(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx, const float *y,
                            int64_t incy, float *d_result) {
  return reduce_to_device<SdotOp>(ctx, n, x, incx, y, incy, d_result, 0.0f, "sdot");
}

extern "C" int wgb_sdot(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx, const float *y,
                        int64_t incy, float *result) {
  return reduce_to_host<SdotOp>(ctx, n, x, incx, y, incy, result, 0.0f, "sdot");
}

extern "C" int wgb_sasum_dev(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx,
                             float *d_result) {
  return reduce_to_device<SasumOp>(ctx, n, x, incx, nullptr, 0, d_result, 0.0f, "sasum");
}

extern "C" int wgb_sasum(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx, float *result) {
  return reduce_to_host<SasumOp>(ctx, n, x, incx, nullptr, 0, result, 0.0f, "sasum");
}

extern "C" int wgb_snrm2_dev(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx,
                             float *d_result) {
  return reduce_to_device<Snrm2Op>(ctx, n, x, incx, nullptr, 0, d_result, 0.0f, "snrm2");
}

extern "C" int wgb_snrm2(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx, float *result) {
  return reduce_to_host<Snrm2Op>(ctx, n, x, incx, nullptr, 0, result, 0.0f, "snrm2");
}

extern "C" int wgb_isamax_dev(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx,
                              int64_t *d_result) {
  return reduce_to_device<IsamaxOp>(ctx, n, x, incx, nullptr, 0, d_result, (int64_t)-1, "isamax");
}

extern "C" int wgb_isamax(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx, int64_t *result) {
  return reduce_to_host<IsamaxOp>(ctx, n, x, incx, nullptr, 0, result, (int64_t)-1, "isamax");
}

// ---- fp64 ---------------------------------------------------------------

extern "C" int wgb_ddot_dev(wgb_ctx *ctx, int64_t n, const double *x, int64_t incx,
                            const double *y, int64_t incy, double *d_result) {
  return reduce_to_device<DdotOp>(ctx, n, x, incx, y, incy, d_result, 0.0, "ddot");
}

extern "C" int wgb_ddot(wgb_ctx *ctx, int64_t n, const double *x, int64_t incx, const double *y,
                        int64_t incy, double *result) {
  return reduce_to_host<DdotOp>(ctx, n, x, incx, y, incy, result, 0.0, "ddot");
}

extern "C" int wgb_dasum_dev(wgb_ctx *ctx, int64_t n, const double *x, int64_t incx,
                             double *d_result) {
  return reduce_to_device<DasumOp>(ctx, n, x, incx, nullptr, 0, d_result, 0.0, "dasum");
}

extern "C" int wgb_dasum(wgb_ctx *ctx, int64_t n, const double *x, int64_t incx, double *result) {
  return reduce_to_host<DasumOp>(ctx, n, x, incx, nullptr, 0, result, 0.0, "dasum");
}

extern "C" int wgb_dnrm2_dev(wgb_ctx *ctx, int64_t n, const double *x, int64_t incx,
                             double *d_result) {
  return reduce_to_device<Dnrm2Op>(ctx, n, x, incx, nullptr, 0, d_result, 0.0, "dnrm2");
}

extern "C" int wgb_dnrm2(wgb_ctx *ctx, int64_t n, const double *x, int64_t incx, double *result) {
  return reduce_to_host<Dnrm2Op>(ctx, n, x, incx, nullptr, 0, result, 0.0, "dnrm2");
}

extern "C" int wgb_idamax_dev(wgb_ctx *ctx, int64_t n, const double *x, int64_t incx,
                              int64_t *d_result) {
  return reduce_to_device<IdamaxOp>(ctx, n, x, incx, nullptr, 0, d_result, (int64_t)-1, "idamax");
}

extern "C" int wgb_idamax(wgb_ctx *ctx, int64_t n, const double *x, int64_t incx,
                          int64_t *result) {
  return reduce_to_host<IdamaxOp>(ctx, n, x, incx, nullptr, 0, result, (int64_t)-1, "idamax");
}
