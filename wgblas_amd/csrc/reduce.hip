// Level-1 reductions: sdot, sasum, snrm2, isamax.
//
// wgblas runs each of these as two compute passes on one encoder: 128
// workgroups of 64 threads grid-stride over x with four accumulators each,
// then a single workgroup folds the 128 partials (src/sdot/sdot.mjs:86-92,
// src/shaders/sdot.wgsl, src/shaders/reduction/sum.wgsl). This file keeps the
// two-pass structure and its determinism, but sizes pass 1 for MI355X's HBM:
//
//  * pass 1 uses G = min(2048, ceil(n / 4096)) blocks of 256 threads; G
//    depends only on n, so the summation order (and the result) is the same
//    on every run and every device;
//  * unit-stride, 16-byte-aligned operands are read as 16-byte vectors, eight loads in
//    flight per lane per iteration; other strides read one element per lane;
//  * a block folds its lanes with 64-lane shuffles, then its four waves in
//    LDS, in a fixed order, and writes one partial;
//  * pass 2 (one block) folds the G partials in a fixed order and, for snrm2
//    and isamax, applies the final combine.
//
// The per-element arithmetic follows the WGSL kernels: f32 accumulation,
// snrm2's big/medium/small classification with the same power-of-two
// thresholds and scales (src/shaders/snrm2.wgsl:33-51), LAPACK 3.10's combine
// (src/shaders/reduction/scaledSum.wgsl:50-101), and isamax's strict '>'
// with a -1 sentinel and lower-index tie break (src/shaders/isamax.wgsl:28-80,
// src/shaders/reduction/argmax.wgsl).
#include "common.h"

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kUnroll = 8;
constexpr int64_t kElemsPerBlockMin = 4096;

// snrm2 thresholds and scales (powers of two): src/shaders/snrm2.wgsl:33-36.
constexpr float kTsml = 0x1p-63f;
constexpr float kTbig = 0x1p50f;
constexpr float kSsml = 0x1p75f;
constexpr float kSbig = 0x1p-76f;
constexpr int kSbigSqExp = -152;  // log2(SBIG^2)

int reduce_blocks(int64_t n) {
  int64_t g = (n + kElemsPerBlockMin - 1) / kElemsPerBlockMin;
  if (g > wgb::kMaxReduceBlocks) g = wgb::kMaxReduceBlocks;
  if (g < 1) g = 1;
  return (int)g;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// ---- wave / block folds (fixed order) ------------------------------------

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Folds one float per thread into thread 0's return value.
__device__ __forceinline__ float block_sum(float v, float *lds) {
  v = wave_sum(v);
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) lds[wave] = v;
  __syncthreads();
  float r = 0.0f;
  if (threadIdx.x == 0) r = (lds[0] + lds[1]) + (lds[2] + lds[3]);
  return r;
}

// isamax's pair order: b replaces a when larger, or equal with a lower index.
__device__ __forceinline__ void amax_merge(float &av, int64_t &ai, float bv, int64_t bi) {
  if (bv > av || (bv == av && bi < ai)) {
    av = bv;
    ai = bi;
  }
}

__device__ __forceinline__ void wave_amax(float &v, int64_t &i) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    float ov = __shfl_xor(v, off, 64);
    int64_t oi = __shfl_xor(i, off, 64);
    amax_merge(v, i, ov, oi);
  }
}

__device__ __forceinline__ void block_amax(float &v, int64_t &i, float *lds_v, int64_t *lds_i) {
  wave_amax(v, i);
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    lds_v[wave] = v;
    lds_i[wave] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    v = lds_v[0];
    i = lds_i[0];
    for (int w = 1; w < kThreads / 64; ++w) amax_merge(v, i, lds_v[w], lds_i[w]);
  }
}

// ---- sdot / sasum ---------------------------------------------------------

__global__ __launch_bounds__(kThreads) void sdot_pass1_vec(const float *__restrict__ x,
                                                           const float *__restrict__ y, int64_t n,
                                                           float *__restrict__ partials) {
  __shared__ float lds[kThreads / 64];
  const v4f *x4 = reinterpret_cast<const v4f *>(x);
  const v4f *y4 = reinterpret_cast<const v4f *>(y);
  const int64_t n4 = n >> 2;
  const int64_t S = (int64_t)gridDim.x * kThreads;
  int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
  for (; q + (kUnroll - 1) * S < n4; q += kUnroll * S) {
    v4f a[kUnroll], b[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      a[u] = __builtin_nontemporal_load(&x4[q + u * S]);
      b[u] = __builtin_nontemporal_load(&y4[q + u * S]);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      acc.x = fmaf(a[u].x, b[u].x, acc.x);
      acc.y = fmaf(a[u].y, b[u].y, acc.y);
      acc.z = fmaf(a[u].z, b[u].z, acc.z);
      acc.w = fmaf(a[u].w, b[u].w, acc.w);
    }
  }
  for (; q < n4; q += S) {
    v4f a = x4[q], b = y4[q];
    acc.x = fmaf(a.x, b.x, acc.x);
    acc.y = fmaf(a.y, b.y, acc.y);
    acc.z = fmaf(a.z, b.z, acc.z);
    acc.w = fmaf(a.w, b.w, acc.w);
  }
  if (blockIdx.x == 0 && threadIdx.x == 0)
    for (int64_t i = n4 * 4; i < n; ++i) acc.x = fmaf(x[i], y[i], acc.x);
  float r = block_sum((acc.x + acc.y) + (acc.z + acc.w), lds);
  if (threadIdx.x == 0) partials[blockIdx.x] = r;
}

__global__ __launch_bounds__(kThreads) void sdot_pass1_strided(const float *__restrict__ x,
                                                               int64_t incx,
                                                               const float *__restrict__ y,
                                                               int64_t incy, int64_t n,
                                                               float *__restrict__ partials) {
  __shared__ float lds[kThreads / 64];
  const int64_t S = (int64_t)gridDim.x * kThreads;
  int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (; i + (kUnroll - 1) * S < n; i += kUnroll * S) {
    float a[kUnroll], b[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      a[u] = x[(i + u * S) * incx];
      b[u] = y[(i + u * S) * incy];
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc[u & 3] = fmaf(a[u], b[u], acc[u & 3]);
  }
  for (; i < n; i += S) acc[0] = fmaf(x[i * incx], y[i * incy], acc[0]);
  float r = block_sum((acc[0] + acc[1]) + (acc[2] + acc[3]), lds);
  if (threadIdx.x == 0) partials[blockIdx.x] = r;
}

__global__ __launch_bounds__(kThreads) void sasum_pass1_vec(const float *__restrict__ x, int64_t n,
                                                            float *__restrict__ partials) {
  __shared__ float lds[kThreads / 64];
  const v4f *x4 = reinterpret_cast<const v4f *>(x);
  const int64_t n4 = n >> 2;
  const int64_t S = (int64_t)gridDim.x * kThreads;
  int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
  for (; q + (kUnroll - 1) * S < n4; q += kUnroll * S) {
    v4f a[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) a[u] = __builtin_nontemporal_load(&x4[q + u * S]);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      acc.x += fabsf(a[u].x);
      acc.y += fabsf(a[u].y);
      acc.z += fabsf(a[u].z);
      acc.w += fabsf(a[u].w);
    }
  }
  for (; q < n4; q += S) {
    v4f a = x4[q];
    acc.x += fabsf(a.x);
    acc.y += fabsf(a.y);
    acc.z += fabsf(a.z);
    acc.w += fabsf(a.w);
  }
  if (blockIdx.x == 0 && threadIdx.x == 0)
    for (int64_t i = n4 * 4; i < n; ++i) acc.x += fabsf(x[i]);
  float r = block_sum((acc.x + acc.y) + (acc.z + acc.w), lds);
  if (threadIdx.x == 0) partials[blockIdx.x] = r;
}

__global__ __launch_bounds__(kThreads) void sasum_pass1_strided(const float *__restrict__ x,
                                                                int64_t incx, int64_t n,
                                                                float *__restrict__ partials) {
  __shared__ float lds[kThreads / 64];
  const int64_t S = (int64_t)gridDim.x * kThreads;
  int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (; i + (kUnroll - 1) * S < n; i += kUnroll * S) {
    float a[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) a[u] = x[(i + u * S) * incx];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc[u & 3] += fabsf(a[u]);
  }
  for (; i < n; i += S) acc[0] += fabsf(x[i * incx]);
  float r = block_sum((acc[0] + acc[1]) + (acc[2] + acc[3]), lds);
  if (threadIdx.x == 0) partials[blockIdx.x] = r;
}

// Pass 2 for sdot/sasum: one block folds G partials in a fixed order.
__global__ __launch_bounds__(kThreads) void sum_pass2(const float *__restrict__ partials, int G,
                                                      float *__restrict__ out) {
  __shared__ float lds[kThreads / 64];
  float acc = 0.0f;
  for (int i = threadIdx.x; i < G; i += kThreads) acc += partials[i];
  float r = block_sum(acc, lds);
  if (threadIdx.x == 0) *out = r;
}

// ---- snrm2 ----------------------------------------------------------------

struct Nrm {
  float big, med, sml;
};

// Adds |v|'s contribution to (big, medium, small) as snrm2.wgsl's accum()
// does: NaN fails both tests and lands in medium, which the combine turns
// into a NaN result.
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

// True when |v| is outside the medium band and not zero (zero adds nothing
// to whichever sum it lands in, so it can take the medium fast path).
__device__ __forceinline__ bool nrm_odd(float v) {
  float ax = fabsf(v);
  return !(ax <= kTbig) || (ax < kTsml && ax != 0.0f);
}

__device__ __forceinline__ void nrm_accum4(Nrm &s, v4f a) {
  bool odd = nrm_odd(a.x) || nrm_odd(a.y) || nrm_odd(a.z) || nrm_odd(a.w);
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

__device__ __forceinline__ void block_nrm(Nrm &s, v4f *lds) {
  s.big = wave_sum(s.big);
  s.med = wave_sum(s.med);
  s.sml = wave_sum(s.sml);
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) lds[wave] = v4f{s.big, s.med, s.sml, 0.f};
  __syncthreads();
  if (threadIdx.x == 0) {
    v4f a = lds[0], b = lds[1], c = lds[2], d = lds[3];
    s.big = (a.x + b.x) + (c.x + d.x);
    s.med = (a.y + b.y) + (c.y + d.y);
    s.sml = (a.z + b.z) + (c.z + d.z);
  }
}

__global__ __launch_bounds__(kThreads) void snrm2_pass1_vec(const float *__restrict__ x, int64_t n,
                                                            v4f *__restrict__ partials) {
  __shared__ v4f lds[kThreads / 64];
  const v4f *x4 = reinterpret_cast<const v4f *>(x);
  const int64_t n4 = n >> 2;
  const int64_t S = (int64_t)gridDim.x * kThreads;
  int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  Nrm s{0.f, 0.f, 0.f};
  for (; q + (kUnroll - 1) * S < n4; q += kUnroll * S) {
    v4f a[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) a[u] = __builtin_nontemporal_load(&x4[q + u * S]);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) nrm_accum4(s, a[u]);
  }
  for (; q < n4; q += S) nrm_accum4(s, x4[q]);
  if (blockIdx.x == 0 && threadIdx.x == 0)
    for (int64_t i = n4 * 4; i < n; ++i) nrm_accum(s, x[i]);
  block_nrm(s, lds);
  if (threadIdx.x == 0) partials[blockIdx.x] = v4f{s.big, s.med, s.sml, 0.f};
}

__global__ __launch_bounds__(kThreads) void snrm2_pass1_strided(const float *__restrict__ x,
                                                                int64_t incx, int64_t n,
                                                                v4f *__restrict__ partials) {
  __shared__ v4f lds[kThreads / 64];
  const int64_t S = (int64_t)gridDim.x * kThreads;
  int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  Nrm s{0.f, 0.f, 0.f};
  for (; i + 3 * S < n; i += 4 * S) {
    v4f a = v4f{x[i * incx], x[(i + S) * incx], x[(i + 2 * S) * incx],
                           x[(i + 3 * S) * incx]};
    nrm_accum4(s, a);
  }
  for (; i < n; i += S) nrm_accum(s, x[i * incx]);
  block_nrm(s, lds);
  if (threadIdx.x == 0) partials[blockIdx.x] = v4f{s.big, s.med, s.sml, 0.f};
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

// LAPACK 3.10 combine of the three sums (scaledSum.wgsl:159-196).
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

__global__ __launch_bounds__(kThreads) void snrm2_pass2(const v4f *__restrict__ partials, int G,
                                                        float *__restrict__ out) {
  __shared__ v4f lds[kThreads / 64];
  Nrm s{0.f, 0.f, 0.f};
  for (int i = threadIdx.x; i < G; i += kThreads) {
    v4f p = partials[i];
    s.big += p.x;
    s.med += p.y;
    s.sml += p.z;
  }
  block_nrm(s, lds);
  if (threadIdx.x == 0) *out = nrm_combine(s.big, s.med, s.sml);
}

// ---- isamax ---------------------------------------------------------------

struct AmaxPartial {
  float val;
  float pad;
  int64_t idx;
};

__device__ __forceinline__ void amax_step(float &best, int64_t &bi, float v, int64_t i) {
  float ax = fabsf(v);
  if (ax > best) {
    best = ax;
    bi = i;
  }
}

__global__ __launch_bounds__(kThreads) void isamax_pass1_vec(const float *__restrict__ x, int64_t n,
                                                             AmaxPartial *__restrict__ partials) {
  __shared__ float lds_v[kThreads / 64];
  __shared__ int64_t lds_i[kThreads / 64];
  const v4f *x4 = reinterpret_cast<const v4f *>(x);
  const int64_t n4 = n >> 2;
  const int64_t S = (int64_t)gridDim.x * kThreads;
  int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  float best = -1.0f;
  int64_t bi = 0;
  for (; q + (kUnroll - 1) * S < n4; q += kUnroll * S) {
    v4f a[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) a[u] = __builtin_nontemporal_load(&x4[q + u * S]);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      int64_t base = (q + u * S) * 4;
      amax_step(best, bi, a[u].x, base);
      amax_step(best, bi, a[u].y, base + 1);
      amax_step(best, bi, a[u].z, base + 2);
      amax_step(best, bi, a[u].w, base + 3);
    }
  }
  for (; q < n4; q += S) {
    v4f a = x4[q];
    int64_t base = q * 4;
    amax_step(best, bi, a.x, base);
    amax_step(best, bi, a.y, base + 1);
    amax_step(best, bi, a.z, base + 2);
    amax_step(best, bi, a.w, base + 3);
  }
  if (blockIdx.x == 0 && threadIdx.x == 0)
    for (int64_t i = n4 * 4; i < n; ++i) amax_step(best, bi, x[i], i);
  block_amax(best, bi, lds_v, lds_i);
  if (threadIdx.x == 0) partials[blockIdx.x] = AmaxPartial{best, 0.f, bi};
}

__global__ __launch_bounds__(kThreads) void isamax_pass1_strided(const float *__restrict__ x,
                                                                 int64_t incx, int64_t n,
                                                                 AmaxPartial *__restrict__ partials) {
  __shared__ float lds_v[kThreads / 64];
  __shared__ int64_t lds_i[kThreads / 64];
  const int64_t S = (int64_t)gridDim.x * kThreads;
  int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  float best = -1.0f;
  int64_t bi = 0;
  for (; i + (kUnroll - 1) * S < n; i += kUnroll * S) {
    float a[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) a[u] = x[(i + u * S) * incx];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) amax_step(best, bi, a[u], i + u * S);
  }
  for (; i < n; i += S) amax_step(best, bi, x[i * incx], i);
  block_amax(best, bi, lds_v, lds_i);
  if (threadIdx.x == 0) partials[blockIdx.x] = AmaxPartial{best, 0.f, bi};
}

__global__ __launch_bounds__(kThreads) void isamax_pass2(const AmaxPartial *__restrict__ partials,
                                                         int G, int64_t *__restrict__ out) {
  __shared__ float lds_v[kThreads / 64];
  __shared__ int64_t lds_i[kThreads / 64];
  float best = -1.0f;
  int64_t bi = 0;
  for (int i = threadIdx.x; i < G; i += kThreads) {
    AmaxPartial p = partials[i];
    amax_merge(best, bi, p.val, p.idx);
  }
  block_amax(best, bi, lds_v, lds_i);
  if (threadIdx.x == 0) *out = bi;
}

// Writes the n <= 0 answer of a `_dev` call with a kernel rather than a
// memset, so the call stays safe to capture in a HIP graph.
template <typename T>
__global__ void set_value(T *out, T v) {
  *out = v;
}

// ---- host side -------------------------------------------------------------

int check_vec(int64_t n, const float *x, int64_t incx, const char *xname, const char *incname) {
  if (incx <= 0)
    return wgb::fail(WGB_ERR_INVALID_VALUE, std::string(incname) + " must be positive");
  if (n > 0 && !x) return wgb::fail(WGB_ERR_INVALID_VALUE, std::string(xname) + " is null");
  return WGB_OK;
}

void *partials_of(wgb_ctx *ctx) { return ctx->scratch; }
void *result_slot(wgb_ctx *ctx) { return (char *)ctx->scratch + (size_t)wgb::kMaxReduceBlocks * 16; }

int launch_sdot(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx, const float *y,
                int64_t incy, float *d_out) {
  int G = reduce_blocks(n);
  float *part = (float *)partials_of(ctx);
  if (incx == 1 && incy == 1 && aligned16(x) && aligned16(y))
    sdot_pass1_vec<<<G, kThreads, 0, ctx->stream>>>(x, y, n, part);
  else
    sdot_pass1_strided<<<G, kThreads, 0, ctx->stream>>>(x, incx, y, incy, n, part);
  WGB_CHECK_LAUNCH("sdot pass 1");
  sum_pass2<<<1, kThreads, 0, ctx->stream>>>(part, G, d_out);
  WGB_CHECK_LAUNCH("sdot pass 2");
  return WGB_OK;
}

int launch_sasum(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx, float *d_out) {
  int G = reduce_blocks(n);
  float *part = (float *)partials_of(ctx);
  if (incx == 1 && aligned16(x))
    sasum_pass1_vec<<<G, kThreads, 0, ctx->stream>>>(x, n, part);
  else
    sasum_pass1_strided<<<G, kThreads, 0, ctx->stream>>>(x, incx, n, part);
  WGB_CHECK_LAUNCH("sasum pass 1");
  sum_pass2<<<1, kThreads, 0, ctx->stream>>>(part, G, d_out);
  WGB_CHECK_LAUNCH("sasum pass 2");
  return WGB_OK;
}

int launch_snrm2(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx, float *d_out) {
  int G = reduce_blocks(n);
  v4f *part = (v4f *)partials_of(ctx);
  if (incx == 1 && aligned16(x))
    snrm2_pass1_vec<<<G, kThreads, 0, ctx->stream>>>(x, n, part);
  else
    snrm2_pass1_strided<<<G, kThreads, 0, ctx->stream>>>(x, incx, n, part);
  WGB_CHECK_LAUNCH("snrm2 pass 1");
  snrm2_pass2<<<1, kThreads, 0, ctx->stream>>>(part, G, d_out);
  WGB_CHECK_LAUNCH("snrm2 pass 2");
  return WGB_OK;
}

int launch_isamax(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx, int64_t *d_out) {
  int G = reduce_blocks(n);
  AmaxPartial *part = (AmaxPartial *)partials_of(ctx);
  if (incx == 1 && aligned16(x))
    isamax_pass1_vec<<<G, kThreads, 0, ctx->stream>>>(x, n, part);
  else
    isamax_pass1_strided<<<G, kThreads, 0, ctx->stream>>>(x, incx, n, part);
  WGB_CHECK_LAUNCH("isamax pass 1");
  isamax_pass2<<<1, kThreads, 0, ctx->stream>>>(part, G, d_out);
  WGB_CHECK_LAUNCH("isamax pass 2");
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

}  // namespace

extern "C" int wgb_sdot_dev(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx, const float *y,
                            int64_t incy, float *d_result) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_vec(n, x, incx, "x", "incx"))) return st;
  if ((st = check_vec(n, y, incy, "y", "incy"))) return st;
  if (!d_result) return wgb::fail(WGB_ERR_INVALID_VALUE, "d_result is null");
  wgb::timing_begin(ctx);
  if (n <= 0)
    set_value<<<1, 1, 0, ctx->stream>>>(d_result, 0.0f);
  else if ((st = launch_sdot(ctx, n, x, incx, y, incy, d_result)))
    return st;
  wgb::timing_end(ctx);
  return WGB_OK;
}

extern "C" int wgb_sdot(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx, const float *y,
                        int64_t incy, float *result) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_vec(n, x, incx, "x", "incx"))) return st;
  if ((st = check_vec(n, y, incy, "y", "incy"))) return st;
  if (!result) return wgb::fail(WGB_ERR_INVALID_VALUE, "result is null");
  if (n <= 0) {
    *result = 0.0f;
    return WGB_OK;
  }
  float *slot = (float *)result_slot(ctx);
  wgb::timing_begin(ctx);
  if ((st = launch_sdot(ctx, n, x, incx, y, incy, slot))) return st;
  wgb::timing_end(ctx);
  return fetch_scalar(ctx, slot, result);
}

extern "C" int wgb_sasum_dev(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx,
                             float *d_result) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_vec(n, x, incx, "x", "incx"))) return st;
  if (!d_result) return wgb::fail(WGB_ERR_INVALID_VALUE, "d_result is null");
  wgb::timing_begin(ctx);
  if (n <= 0)
    set_value<<<1, 1, 0, ctx->stream>>>(d_result, 0.0f);
  else if ((st = launch_sasum(ctx, n, x, incx, d_result)))
    return st;
  wgb::timing_end(ctx);
  return WGB_OK;
}

extern "C" int wgb_sasum(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx, float *result) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_vec(n, x, incx, "x", "incx"))) return st;
  if (!result) return wgb::fail(WGB_ERR_INVALID_VALUE, "result is null");
  if (n <= 0) {
    *result = 0.0f;
    return WGB_OK;
  }
  float *slot = (float *)result_slot(ctx);
  wgb::timing_begin(ctx);
  if ((st = launch_sasum(ctx, n, x, incx, slot))) return st;
  wgb::timing_end(ctx);
  return fetch_scalar(ctx, slot, result);
}

extern "C" int wgb_snrm2_dev(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx,
                             float *d_result) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_vec(n, x, incx, "x", "incx"))) return st;
  if (!d_result) return wgb::fail(WGB_ERR_INVALID_VALUE, "d_result is null");
  wgb::timing_begin(ctx);
  if (n <= 0)
    set_value<<<1, 1, 0, ctx->stream>>>(d_result, 0.0f);
  else if ((st = launch_snrm2(ctx, n, x, incx, d_result)))
    return st;
  wgb::timing_end(ctx);
  return WGB_OK;
}

extern "C" int wgb_snrm2(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx, float *result) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_vec(n, x, incx, "x", "incx"))) return st;
  if (!result) return wgb::fail(WGB_ERR_INVALID_VALUE, "result is null");
  if (n <= 0) {
    *result = 0.0f;
    return WGB_OK;
  }
  float *slot = (float *)result_slot(ctx);
  wgb::timing_begin(ctx);
  if ((st = launch_snrm2(ctx, n, x, incx, slot))) return st;
  wgb::timing_end(ctx);
  return fetch_scalar(ctx, slot, result);
}

extern "C" int wgb_isamax_dev(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx,
                              int64_t *d_result) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_vec(n, x, incx, "x", "incx"))) return st;
  if (!d_result) return wgb::fail(WGB_ERR_INVALID_VALUE, "d_result is null");
  wgb::timing_begin(ctx);
  if (n <= 0)
    set_value<<<1, 1, 0, ctx->stream>>>(d_result, (int64_t)-1);
  else if ((st = launch_isamax(ctx, n, x, incx, d_result)))
    return st;
  wgb::timing_end(ctx);
  return WGB_OK;
}

extern "C" int wgb_isamax(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx, int64_t *result) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if ((st = check_vec(n, x, incx, "x", "incx"))) return st;
  if (!result) return wgb::fail(WGB_ERR_INVALID_VALUE, "result is null");
  if (n <= 0) {
    *result = -1;
    return WGB_OK;
  }
  int64_t *slot = (int64_t *)result_slot(ctx);
  wgb::timing_begin(ctx);
  if ((st = launch_isamax(ctx, n, x, incx, slot))) return st;
  wgb::timing_end(ctx);
  return fetch_scalar(ctx, slot, result);
}
