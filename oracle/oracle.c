/*
 * oracle.c — CPU restatement of wgblas's hot path, used ONLY as the checker
 * in tests, in __graft_entry__.smoke() and in bench.py's cpu_baseline leg.
 * Nothing in the product (wgblas_amd/) links, loads or calls this file.
 *
 * Two kinds of functions live here:
 *
 *  1. "wgsl" restatements: the reference's own arithmetic order, in IEEE
 *     float32, so they reproduce what wgblas's WGSL kernels compute (up to a
 *     shader compiler's choice to fuse a multiply-add):
 *       orc_random_f32/f64  src/random/random.mjs:4-26 (mulberry32)
 *       orc_sdot_wgsl       src/shaders/sdot.wgsl:19-53 + reduction/sum.wgsl:12-26,
 *                           dispatch src/sdot/sdot.mjs:89-92 (2*WGS workgroups of WGS=64)
 *       orc_sasum_wgsl      src/shaders/sasum.wgsl:17-51 + reduction/sum.wgsl
 *       orc_snrm2_wgsl      src/shaders/snrm2.wgsl:33-95 + reduction/scaledSum.wgsl:32-101
 *       orc_isamax_wgsl     src/shaders/isamax.wgsl:19-82 + reduction/argmax.wgsl:14-43
 *       orc_sgemm_wgsl      src/shaders/sgemm_large.wgsl:112-308 per-element order
 *                           (sequential k, then alpha*acc, then + beta*C, masks)
 *
 *  2. extended-precision references that the error bounds are measured
 *     against: orc_gemm_ld (long double accumulation, any uplo/trans, with the
 *     reference's alpha/beta rules of sgemm_large.wgsl:299-304 and
 *     dgemm.mjs:177-179), orc_dot_ld, orc_sum_abs_ld, orc_nrm2_ld,
 *     orc_isamax_brute (first index of max |x|, NaN skipped).
 *
 * The normal(0,1) sampler (orc_random_normal_f32) restates the sampler this
 * build defines (include/wgblas_hip.h, wgb_fill_normal_f32); the reference
 * has none.
 *
 * Matrices are column-major with a leading dimension, as in the C ABI.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define WGS 64
#define NWG (2 * WGS)

/* ---- mulberry32 (src/random/random.mjs:4-12) ---------------------------- */

static uint32_t mulberry_next(uint32_t *state) {
  uint32_t a = *state + 0x6d2b79f5u;
  *state = a;
  uint32_t t = (a ^ (a >> 15)) * (1u | a);
  t = (t + (t ^ (t >> 7)) * (61u | t)) ^ t;
  return t ^ (t >> 14);
}

/* randomFloat32Array(n, low, high, seed): low + next()*(high-low) in double,
 * stored to float32 (src/random/random.mjs:14-19). */
void orc_random_f32(int64_t n, double low, double high, uint32_t seed, float *out) {
  uint32_t s = seed;
  volatile double range = high - low;
  for (int64_t i = 0; i < n; ++i) {
    volatile double u = (double)mulberry_next(&s) / 4294967296.0;
    volatile double prod = u * range;
    out[i] = (float)(low + prod);
  }
}

void orc_random_f64(int64_t n, double low, double high, uint32_t seed, double *out) {
  uint32_t s = seed;
  volatile double range = high - low;
  for (int64_t i = 0; i < n; ++i) {
    volatile double u = (double)mulberry_next(&s) / 4294967296.0;
    volatile double prod = u * range;
    out[i] = low + prod;
  }
}

/* The build's normal(0,1) sampler: Box-Muller over the mulberry32 stream,
 * pair p from draws 2p and 2p+1, r = sqrt(-2 ln(1-u1)), t = 2 pi u2. */
void orc_random_normal_f32(int64_t n, uint32_t seed, float *out) {
  uint32_t s = seed;
  const double two_pi = 6.283185307179586476925286766559;
  for (int64_t i = 0; i < n; i += 2) {
    double u1 = (double)mulberry_next(&s) / 4294967296.0;
    double u2 = (double)mulberry_next(&s) / 4294967296.0;
    double r = sqrt(-2.0 * log(1.0 - u1));
    double t = two_pi * u2;
    out[i] = (float)(r * cos(t));
    if (i + 1 < n) out[i + 1] = (float)(r * sin(t));
  }
}

/* ---- level-1 reductions in the reference's order -------------------------- */

/* LDS tree over WGS values: for s = 32..1, tile[l] += tile[l+s]. */
static float tree_sum(float *t, int len) {
  for (int s = len / 2; s > 0; s >>= 1)
    for (int l = 0; l < s; ++l) t[l] = t[l] + t[l + s];
  return t[0];
}

/* reduction/sum.wgsl:12-26: tile[i] = p[i] + p[i+WGS], then the tree. */
static float sum_pass2(const float *partials) {
  float tile[WGS];
  for (int i = 0; i < WGS; ++i) tile[i] = partials[i] + partials[i + WGS];
  return tree_sum(tile, WGS);
}

float orc_sdot_wgsl(int64_t n, const float *x, int64_t incx, const float *y, int64_t incy) {
  if (n <= 0) return 0.0f; /* src/sdot/sdot.mjs:40 */
  float partials[NWG];
  float tile[WGS];
  const int64_t stride = (int64_t)NWG * WGS;
  const int64_t n4_floor = (n / (4 * stride)) * (4 * stride);
  for (int w = 0; w < NWG; ++w) {
    for (int l = 0; l < WGS; ++l) {
      int64_t gid = (int64_t)w * WGS + l;
      float a0 = 0, a1 = 0, a2 = 0, a3 = 0;
      for (int64_t id = gid; id < n4_floor; id += 4 * stride) {
        a0 += x[id * incx] * y[id * incy];
        a1 += x[(id + stride) * incx] * y[(id + stride) * incy];
        a2 += x[(id + 2 * stride) * incx] * y[(id + 2 * stride) * incy];
        a3 += x[(id + 3 * stride) * incx] * y[(id + 3 * stride) * incy];
      }
      for (int64_t id = n4_floor + gid; id < n; id += stride) a0 += x[id * incx] * y[id * incy];
      tile[l] = a0 + a1 + a2 + a3;
    }
    partials[w] = tree_sum(tile, WGS);
  }
  return sum_pass2(partials);
}

float orc_sasum_wgsl(int64_t n, const float *x, int64_t incx) {
  if (n <= 0) return 0.0f; /* src/sasum/sasum.mjs:28 */
  float partials[NWG];
  float tile[WGS];
  const int64_t stride = (int64_t)NWG * WGS;
  const int64_t n4_floor = (n / (4 * stride)) * (4 * stride);
  for (int w = 0; w < NWG; ++w) {
    for (int l = 0; l < WGS; ++l) {
      int64_t gid = (int64_t)w * WGS + l;
      float a0 = 0, a1 = 0, a2 = 0, a3 = 0;
      for (int64_t id = gid; id < n4_floor; id += 4 * stride) {
        a0 += fabsf(x[id * incx]);
        a1 += fabsf(x[(id + stride) * incx]);
        a2 += fabsf(x[(id + 2 * stride) * incx]);
        a3 += fabsf(x[(id + 3 * stride) * incx]);
      }
      for (int64_t id = n4_floor + gid; id < n; id += stride) a0 += fabsf(x[id * incx]);
      tile[l] = a0 + a1 + a2 + a3;
    }
    partials[w] = tree_sum(tile, WGS);
  }
  return sum_pass2(partials);
}

/* snrm2.wgsl:33-36 */
#define TSML 0x1p-63f
#define TBIG 0x1p50f
#define SSML 0x1p75f
#define SBIG 0x1p-76f

typedef struct {
  float big, med, sml;
} nrm3;

/* snrm2.wgsl:40-51 accum(): NaN fails both tests and lands in medium. */
static nrm3 nrm_accum(nrm3 s, float xi) {
  float ax = fabsf(xi);
  int big = ax > TBIG;
  int sml = ax < TSML;
  float yb = ax * SBIG;
  float ys = ax * SSML;
  nrm3 r;
  r.big = s.big + (big ? yb * yb : 0.0f);
  r.med = s.med + ((big || sml) ? 0.0f : ax * ax);
  r.sml = s.sml + (sml ? ys * ys : 0.0f);
  return r;
}

static nrm3 nrm_add(nrm3 a, nrm3 b) {
  nrm3 r = {a.big + b.big, a.med + b.med, a.sml + b.sml};
  return r;
}

/* scaledSum.wgsl:20-24 (NaN test on the bit pattern) */
static int is_nan_bits(float v) {
  uint32_t b;
  memcpy(&b, &v, 4);
  return (b & 0x7fffffffu) > 0x7f800000u;
}

static float ldexp_bits(float v, int e) {
  uint32_t bits;
  memcpy(&bits, &v, 4);
  uint32_t sign = bits & 0x80000000u;
  int ev = (int)((bits >> 23) & 0xffu);
  if (ev == 255) return v;
  int en = ev + e;
  uint32_t out;
  if (ev == 0 || en <= 0) out = sign;
  else if (en >= 255) out = sign | 0x7f800000u;
  else out = (bits & 0x807fffffu) | ((uint32_t)en << 23);
  float r;
  memcpy(&r, &out, 4);
  return r;
}

/* scaledSum.wgsl:64-101: the LAPACK 3.10 combine. */
float orc_nrm_combine(float abig, float amed, float asml) {
  if (is_nan_bits(amed)) return amed;
  int med_live = amed > 0.0f;
  float scl = 1.0f;
  float sumsq = amed;
  if (abig > 0.0f) {
    if (med_live) abig = abig + ldexp_bits(amed, -152);
    scl = 1.0f / SBIG;
    sumsq = abig;
  } else if (asml > 0.0f) {
    if (med_live) {
      amed = sqrtf(amed);
      asml = sqrtf(asml) / SSML;
      float ymax = asml > amed ? asml : amed;
      float ymin = asml < amed ? asml : amed;
      float q = ymin / ymax;
      sumsq = ymax * ymax * (1.0f + q * q);
    } else {
      scl = 1.0f / SSML;
      sumsq = asml;
    }
  }
  return scl * sqrtf(sumsq);
}

float orc_snrm2_wgsl(int64_t n, const float *x, int64_t incx) {
  if (n <= 0) return 0.0f; /* src/snrm2/snrm2.mjs:28 */
  nrm3 partials[NWG];
  nrm3 tile[WGS];
  const int64_t stride = (int64_t)NWG * WGS;
  const int64_t n4_floor = (n / (4 * stride)) * (4 * stride);
  const nrm3 zero = {0, 0, 0};
  for (int w = 0; w < NWG; ++w) {
    for (int l = 0; l < WGS; ++l) {
      int64_t gid = (int64_t)w * WGS + l;
      nrm3 a0 = zero, a1 = zero, a2 = zero, a3 = zero;
      for (int64_t id = gid; id < n4_floor; id += 4 * stride) {
        a0 = nrm_accum(a0, x[id * incx]);
        a1 = nrm_accum(a1, x[(id + stride) * incx]);
        a2 = nrm_accum(a2, x[(id + 2 * stride) * incx]);
        a3 = nrm_accum(a3, x[(id + 3 * stride) * incx]);
      }
      for (int64_t id = n4_floor + gid; id < n; id += stride) a0 = nrm_accum(a0, x[id * incx]);
      tile[l] = nrm_add(nrm_add(a0, a1), nrm_add(a2, a3)); /* snrm2.wgsl:80 */
    }
    for (int s = WGS / 2; s > 0; s >>= 1)
      for (int l = 0; l < s; ++l) tile[l] = nrm_add(tile[l], tile[l + s]);
    partials[w] = tile[0];
  }
  for (int i = 0; i < WGS; ++i) tile[i] = nrm_add(partials[i], partials[i + WGS]);
  for (int s = WGS / 2; s > 0; s >>= 1)
    for (int l = 0; l < s; ++l) tile[l] = nrm_add(tile[l], tile[l + s]);
  return orc_nrm_combine(tile[0].big, tile[0].med, tile[0].sml);
}

/* isamax.wgsl:51-58 / argmax.wgsl: b wins when larger, or equal and lower index. */
static int amax_better(float bv, uint32_t bi, float av, uint32_t ai) {
  return bv > av || (bv == av && bi < ai);
}

int64_t orc_isamax_wgsl(int64_t n, const float *x, int64_t incx) {
  if (n <= 0) return -1; /* src/isamax/isamax.mjs:30 */
  float pv[NWG];
  uint32_t pi[NWG];
  float tv[WGS];
  uint32_t ti[WGS];
  const int64_t stride = (int64_t)NWG * WGS;
  const int64_t n4_floor = (n / (4 * stride)) * (4 * stride);
  for (int w = 0; w < NWG; ++w) {
    for (int l = 0; l < WGS; ++l) {
      int64_t gid = (int64_t)w * WGS + l;
      float bv[4] = {-1.0f, -1.0f, -1.0f, -1.0f};
      uint32_t bi[4] = {0, 0, 0, 0};
      for (int64_t id = gid; id < n4_floor; id += 4 * stride)
        for (int u = 0; u < 4; ++u) {
          float v = fabsf(x[(id + u * stride) * incx]);
          if (v > bv[u]) {
            bv[u] = v;
            bi[u] = (uint32_t)(id + u * stride);
          }
        }
      for (int64_t id = n4_floor + gid; id < n; id += stride) {
        float v = fabsf(x[id * incx]);
        if (v > bv[0]) {
          bv[0] = v;
          bi[0] = (uint32_t)id;
        }
      }
      for (int u = 1; u < 4; ++u)
        if (amax_better(bv[u], bi[u], bv[0], bi[0])) {
          bv[0] = bv[u];
          bi[0] = bi[u];
        }
      tv[l] = bv[0];
      ti[l] = bi[0];
    }
    for (int s = WGS / 2; s > 0; s >>= 1)
      for (int l = 0; l < s; ++l)
        if (amax_better(tv[l + s], ti[l + s], tv[l], ti[l])) {
          tv[l] = tv[l + s];
          ti[l] = ti[l + s];
        }
    pv[w] = tv[0];
    pi[w] = ti[0];
  }
  for (int i = 0; i < WGS; ++i) {
    if (amax_better(pv[i + WGS], pi[i + WGS], pv[i], pi[i])) {
      tv[i] = pv[i + WGS];
      ti[i] = pi[i + WGS];
    } else {
      tv[i] = pv[i];
      ti[i] = pi[i];
    }
  }
  for (int s = WGS / 2; s > 0; s >>= 1)
    for (int l = 0; l < s; ++l)
      if (amax_better(tv[l + s], ti[l + s], tv[l], ti[l])) {
        tv[l] = tv[l + s];
        ti[l] = ti[l + s];
      }
  return (int64_t)ti[0];
}

/* ---- extended-precision references for the bounds ------------------------ */

double orc_dot_ld(int64_t n, const float *x, int64_t incx, const float *y, int64_t incy,
                  double *sum_abs) {
  long double s = 0, a = 0;
  for (int64_t i = 0; i < n; ++i) {
    long double p = (long double)x[i * incx] * (long double)y[i * incy];
    s += p;
    a += fabsl(p);
  }
  if (sum_abs) *sum_abs = (double)a;
  return (double)s;
}

double orc_sum_abs_ld(int64_t n, const float *x, int64_t incx) {
  long double a = 0;
  for (int64_t i = 0; i < n; ++i) a += fabsl((long double)x[i * incx]);
  return (double)a;
}

double orc_nrm2_ld(int64_t n, const float *x, int64_t incx) {
  long double s = 0;
  for (int64_t i = 0; i < n; ++i) {
    long double v = (long double)x[i * incx];
    s += v * v;
  }
  return (double)sqrtl(s);
}

/* First index of max |x|, NaN never selected, all-NaN -> 0, n <= 0 -> -1
 * (src/isamax/isamax.d.mts; tests/isamax/src/test.isamax.js:97-139). */
int64_t orc_isamax_brute(int64_t n, const float *x, int64_t incx) {
  if (n <= 0) return -1;
  int64_t best = 0;
  float bv = -1.0f;
  for (int64_t i = 0; i < n; ++i) {
    float v = fabsf(x[i * incx]);
    if (v > bv) {
      bv = v;
      best = i;
    }
  }
  return best;
}

/* fp64 level 1 (src/ddot/ddot.mjs, src/dasum/dasum.mjs, src/dnrm2/dnrm2.mjs,
 * src/idamax/idamax.mjs): the reference's tests compare with stdlib's f64
 * routines under eps = 2^-48 bounds (tests/ddot/helpers.js,
 * tests/dnrm2/helpers.js) or exactly (idamax); these long-double sums are
 * the exact values those bounds are taken around. */
double orc_ddot_ld(int64_t n, const double *x, int64_t incx, const double *y, int64_t incy,
                   double *sum_abs) {
  long double s = 0, a = 0;
  for (int64_t i = 0; i < n; ++i) {
    long double p = (long double)x[i * incx] * (long double)y[i * incy];
    s += p;
    a += fabsl(p);
  }
  if (sum_abs) *sum_abs = (double)a;
  return (double)s;
}

double orc_dasum_ld(int64_t n, const double *x, int64_t incx) {
  long double a = 0;
  for (int64_t i = 0; i < n; ++i) a += fabsl((long double)x[i * incx]);
  return (double)a;
}

/* long double squares cannot overflow for double inputs (|x|^2 <= 2^2048 is
 * far below long double's 2^16384), so no scaling is needed here. */
double orc_dnrm2_ld(int64_t n, const double *x, int64_t incx) {
  long double s = 0;
  for (int64_t i = 0; i < n; ++i) {
    long double v = (long double)x[i * incx];
    s += v * v;
  }
  return (double)sqrtl(s);
}

/* idamax: isamax's rules on doubles (src/idamax/idamax.mjs:34-36,
 * tests/idamax/src/test.idamax.js:97-126). */
int64_t orc_idamax_brute(int64_t n, const double *x, int64_t incx) {
  if (n <= 0) return -1;
  int64_t best = 0;
  double bv = -1.0;
  for (int64_t i = 0; i < n; ++i) {
    double v = fabs(x[i * incx]);
    if (v > bv) {
      bv = v;
      best = i;
    }
  }
  return best;
}

/* op(M)[r][c] of a column-major matrix with leading dimension ld. */
static inline double op_elem(const double *M, int64_t ld, int trans, int64_t r, int64_t c) {
  return trans ? M[c + r * ld] : M[r + c * ld];
}

/* out (m x n, leading dimension ldo, column-major) <- alpha*op(A)op(B) + beta*C
 * in long double, on the uplo part (0 full, 1 lower i>=j, 2 upper i<=j);
 * elements outside it are copied from C. absdot (may be NULL) receives
 * sum_p |op(A)[i,p]*op(B)[p,j]|. alpha == 0 or k == 0 never reads A or B,
 * beta == 0 never reads C (src/shaders/sgemm_large.wgsl:299-304). */
void orc_gemm_ld(int uplo, int transA, int transB, int64_t m, int64_t n, int64_t k, double alpha,
                 const double *A, int64_t lda, const double *B, int64_t ldb, double beta,
                 const double *C, int64_t ldc, double *out, int64_t ldo, double *absdot) {
  for (int64_t j = 0; j < n; ++j) {
    for (int64_t i = 0; i < m; ++i) {
      int in_tri = uplo == 0 || (uplo == 1 && i >= j) || (uplo == 2 && i <= j);
      if (!in_tri) {
        out[i + j * ldo] = C[i + j * ldc];
        if (absdot) absdot[i + j * ldo] = 0.0;
        continue;
      }
      long double s = 0, a = 0;
      if (alpha != 0.0)
        for (int64_t p = 0; p < k; ++p) {
          long double prod =
              (long double)op_elem(A, lda, transA, i, p) * (long double)op_elem(B, ldb, transB, p, j);
          s += prod;
          a += fabsl(prod);
        }
      long double v = (alpha == 0.0) ? 0.0L : (long double)alpha * s;
      if (beta != 0.0) v += (long double)beta * (long double)C[i + j * ldc];
      out[i + j * ldo] = (double)v;
      if (absdot) absdot[i + j * ldo] = (double)a;
    }
  }
}

/* The reference's per-element fp32 order (sgemm_large.wgsl:221-233, 288-308):
 * acc += a*b sequentially over k (product rounded, then the sum), then
 * alpha*acc, then acc + beta*C; alpha == 0 gives a 0 product term and
 * beta == 0 leaves C unread. Used as the timed CPU baseline. C is updated in
 * place on the uplo part. */
void orc_sgemm_wgsl(int uplo, int transA, int transB, int64_t m, int64_t n, int64_t k,
                    float alpha, const float *A, int64_t lda, const float *B, int64_t ldb,
                    float beta, float *Cm, int64_t ldc) {
  for (int64_t j = 0; j < n; ++j) {
    for (int64_t i = 0; i < m; ++i) {
      int in_tri = uplo == 0 || (uplo == 1 && i >= j) || (uplo == 2 && i <= j);
      if (!in_tri) continue;
      float acc = 0.0f;
      for (int64_t p = 0; p < k; ++p) {
        float a = transA ? A[p + i * lda] : A[i + p * lda];
        float b = transB ? B[j + p * ldb] : B[p + j * ldb];
        volatile float prod = a * b;
        acc = acc + prod;
      }
      float r = alpha == 0.0f ? 0.0f : alpha * acc;
      float *cp = &Cm[i + j * ldc];
      if (beta != 0.0f) {
        volatile float bc = beta * *cp;
        r = r + bc;
      }
      *cp = r;
    }
  }
}

/* ---- level 3 on the GEMM (src/{ssyr2k,ssymm,strmm,strsm}) ----------------
 * The reference's tests compare with stdlib's ssyr2k/ssymm/strmm/strsm
 * (reference BLAS ports) under forward-error bounds (tests/ssyr2k/helpers.js,
 * tests/ssymm/helpers.js, tests/strmm/helpers.js) or a backward residual
 * (tests/strsm/helpers.js). These restate the mathematics in long double:
 * the exact values the bounds are taken around. Matrices are column-major
 * with leading dimensions; sides and diag as in include/wgblas_hip.h
 * (side 1 left / 2 right, uplo 1 lower / 2 upper, diag 1 unit). */

/* C <- alpha*(op(A) op(B)^T + op(B) op(A)^T) + beta*C on the uplo triangle
 * (src/ssyr2k/ssyr2k.mjs:25-26); op(X) is n x k (X n x k stored, trans 0) or
 * X^T. alpha == 0 reads neither A nor B, beta == 0 never reads C.
 * absdot1/absdot2 (may be NULL) get sum_p |op(A)[i,p] op(B)[j,p]| and
 * sum_p |op(B)[i,p] op(A)[j,p]|. Elements outside the triangle keep C. */
void orc_ssyr2k_ld(int uplo, int trans, int64_t n, int64_t k, double alpha, const double *A,
                   int64_t lda, const double *B, int64_t ldb, double beta, const double *C,
                   int64_t ldc, double *out, double *absdot1, double *absdot2) {
  for (int64_t j = 0; j < n; ++j)
    for (int64_t i = 0; i < n; ++i) {
      int64_t o = i + j * ldc;
      int in_tri = uplo == 1 ? i >= j : i <= j;
      if (absdot1) absdot1[o] = 0.0;
      if (absdot2) absdot2[o] = 0.0;
      if (!in_tri) {
        out[o] = C[o];
        continue;
      }
      long double s = 0, a1 = 0, a2 = 0;
      if (alpha != 0.0)
        for (int64_t p = 0; p < k; ++p) {
          /* op(X)[r, p] = X[r + p*ld] (trans 0) or X[p + r*ld] */
          long double ai = trans ? A[p + i * lda] : A[i + p * lda];
          long double aj = trans ? A[p + j * lda] : A[j + p * lda];
          long double bi = trans ? B[p + i * ldb] : B[i + p * ldb];
          long double bj = trans ? B[p + j * ldb] : B[j + p * ldb];
          s += ai * bj + bi * aj;
          a1 += fabsl(ai * bj);
          a2 += fabsl(bi * aj);
        }
      long double v = (long double)alpha * s;
      if (beta != 0.0) v += (long double)beta * C[o];
      out[o] = (double)v;
      if (absdot1) absdot1[o] = (double)a1;
      if (absdot2) absdot2[o] = (double)a2;
    }
}

/* The symmetric matrix whose uplo triangle A stores, element (i, k)
 * (src/shaders/symmetrize.wgsl). */
static inline long double sym_elem(const double *A, int64_t lda, int uplo, int64_t i, int64_t k) {
  int stored = uplo == 1 ? i >= k : i <= k;
  return stored ? A[i + k * lda] : A[k + i * lda];
}

/* C <- alpha*S*B + beta*C (side 1) or alpha*B*S + beta*C (side 2), S the
 * symmetric matrix of A's uplo triangle; C, B m x n (src/ssymm/ssymm.mjs:
 * 27-29). alpha == 0 reads neither A nor B, beta == 0 never reads C. absdot
 * (may be NULL) gets sum_p |S B| terms. */
void orc_ssymm_ld(int side, int uplo, int64_t m, int64_t n, double alpha, const double *A,
                  int64_t lda, const double *B, int64_t ldb, double beta, const double *C,
                  int64_t ldc, double *out, double *absdot) {
  int64_t order = side == 1 ? m : n;
  for (int64_t j = 0; j < n; ++j)
    for (int64_t i = 0; i < m; ++i) {
      long double s = 0, a = 0;
      if (alpha != 0.0)
        for (int64_t p = 0; p < order; ++p) {
          long double t = side == 1 ? sym_elem(A, lda, uplo, i, p) * (long double)B[p + j * ldb]
                                    : (long double)B[i + p * ldb] * sym_elem(A, lda, uplo, p, j);
          s += t;
          a += fabsl(t);
        }
      long double v = (long double)alpha * s;
      if (beta != 0.0) v += (long double)beta * C[i + j * ldc];
      out[i + j * ldc] = (double)v;
      if (absdot) absdot[i + j * ldc] = (double)a;
    }
}

/* op(A)[i, k] of a triangular A: the uplo triangle of A (or of A^T), the
 * diagonal taken as 1 for a unit triangle; *inside is 0 outside the
 * triangle (the structural zeros the sums below skip). */
static inline long double tri_elem(const double *A, int64_t lda, int uplo, int trans, int unit,
                                   int64_t i, int64_t k, int *inside) {
  if (i == k) {
    *inside = 1;
    return unit ? 1.0L : (long double)A[i + i * lda];
  }
  /* op(A) lower iff (uplo lower) != trans */
  int op_lower = (uplo == 1) != (trans != 0);
  *inside = op_lower ? i > k : i < k;
  if (!*inside) return 0.0L;
  return trans ? A[k + i * lda] : A[i + k * lda];
}

/* B <- alpha*op(A)*B (side 1) or alpha*B*op(A) (side 2), A triangular
 * (src/strmm/strmm.mjs:27-29); the sums run over the triangle only, as
 * reference BLAS's loops do. alpha == 0 gives zeros without reading A or B.
 * out has B's layout (ldb); its padding is copied from B. absdot (may be
 * NULL) gets sum_p |op(A) B| terms. */
void orc_strmm_ld(int side, int uplo, int trans, int unit, int64_t m, int64_t n, double alpha,
                  const double *A, int64_t lda, const double *B, int64_t ldb, double *out,
                  double *absdot) {
  int64_t order = side == 1 ? m : n;
  for (int64_t j = 0; j < n; ++j)
    for (int64_t i = 0; i < m; ++i) {
      long double s = 0, a = 0;
      if (alpha != 0.0)
        for (int64_t p = 0; p < order; ++p) {
          int inside;
          long double t;
          if (side == 1) {
            long double e = tri_elem(A, lda, uplo, trans, unit, i, p, &inside);
            if (!inside) continue;
            t = e * (long double)B[p + j * ldb];
          } else {
            long double e = tri_elem(A, lda, uplo, trans, unit, p, j, &inside);
            if (!inside) continue;
            t = (long double)B[i + p * ldb] * e;
          }
          s += t;
          a += fabsl(t);
        }
      out[i + j * ldb] = (double)((long double)alpha * s);
      if (absdot) absdot[i + j * ldb] = (double)a;
    }
}

/* Solves op(A) X = alpha B (side 1) or X op(A) = alpha B (side 2) by
 * substitution in long double (src/strsm/strsm.mjs:148-151). out holds B on
 * entry (ldb) and X on return; padding untouched. Per right-hand side the
 * unknowns go in dependency order, each x = (alpha b - sum of the solved
 * terms in its row) / diagonal, with no zero skipping (as wgblas's strsm).
 * alpha == 0 gives zeros without reading A or B. */
void orc_strsm_ld(int side, int uplo, int trans, int unit, int64_t m, int64_t n, double alpha,
                  const double *A, int64_t lda, double *out, int64_t ldb) {
  int64_t order = side == 1 ? m : n, nrhs = side == 1 ? n : m;
  int op_lower = (uplo == 1) != (trans != 0);
  /* left: unknown i of rhs r is X[i, r], coupled by op(A)[i, k]; forward iff
   * op(A) lower. right: unknown i of rhs r is X[r, i], coupled by
   * op(A)[k, i]; forward iff op(A) upper. */
  int forward = side == 1 ? op_lower : !op_lower;
  for (int64_t r = 0; r < nrhs; ++r) {
    for (int64_t q = 0; q < order; ++q) {
      int64_t i = forward ? q : order - 1 - q;
      double *xi = side == 1 ? &out[i + r * ldb] : &out[r + i * ldb];
      if (alpha == 0.0) {
        *xi = 0.0;
        continue;
      }
      long double s = (long double)alpha * (long double)*xi;
      for (int64_t qq = 0; qq < q; ++qq) {
        int64_t k = forward ? qq : order - 1 - qq;
        int inside;
        long double c = side == 1 ? tri_elem(A, lda, uplo, trans, unit, i, k, &inside)
                                  : tri_elem(A, lda, uplo, trans, unit, k, i, &inside);
        if (!inside) continue;
        long double xk = side == 1 ? out[k + r * ldb] : out[r + k * ldb];
        s -= c * xk;
      }
      int inside;
      long double d = tri_elem(A, lda, uplo, trans, unit, i, i, &inside);
      *xi = (double)(s / d);
    }
  }
}

/* ---- level 2: sgemv (src/sgemv/sgemv.mjs:19-254) -------------------------
 * y <- alpha op(A) x + beta y, A m x n column-major, in long double, with
 * reference BLAS's rules, which the reference's tests hold it to through
 * stdlib (tests/sgemv/src/test.sgemv.js:157-202, 299-387): m == 0, n == 0,
 * or alpha == 0 with beta == 1 leave y untouched; alpha == 0 reads neither A
 * nor x; beta == 0 never reads y; the no-transpose form (column by column)
 * skips a column whose x entry is zero, the transposed (dot-product) form
 * takes every term. absdot (may be NULL, length of y, stride 1) gets
 * sum |a x| over the terms taken. */
void orc_sgemv_ld(int trans, int64_t m, int64_t n, double alpha, const double *A, int64_t lda,
                  const double *x, int64_t incx, double beta, double *y, int64_t incy,
                  double *absdot) {
  int64_t len = trans ? n : m;
  if (absdot)
    for (int64_t i = 0; i < len; ++i) absdot[i] = 0.0;
  if (m == 0 || n == 0 || (alpha == 0.0 && beta == 1.0)) return;
  for (int64_t i = 0; i < len; ++i) {
    long double s = 0, a = 0;
    if (alpha != 0.0) {
      int64_t terms = trans ? m : n;
      for (int64_t p = 0; p < terms; ++p) {
        long double xv = x[p * incx];
        if (!trans && xv == 0.0L) continue;  /* the skipped column */
        long double av = trans ? A[p + i * lda] : A[i + p * lda];
        s += av * xv;
        a += fabsl(av * xv);
      }
    }
    long double v = (long double)alpha * s;
    if (beta != 0.0) v += (long double)beta * y[i * incy];
    y[i * incy] = (double)v;
    if (absdot) absdot[i] = (double)a;
  }
}

/* ---- level 2: sger / dger (src/sger/sger.mjs:17-176, src/dger/dger.mjs) --
 * A <- alpha x y^T + A, A m x n column-major, in long double, with reference
 * BLAS's column order, which the reference's tests hold it to through stdlib
 * (tests/sger/src/test.sger.js:141-178, 219-298): m == 0, n == 0 or
 * alpha == 0 leave A untouched (x and y unread); column j is skipped when
 * y[j] is zero (so Infinity or NaN in x never meets that zero), otherwise
 * A(i, j) += x[i] * (alpha * y[j]) for every row, zeros in x included. In
 * the reference's row-major frame the skipped vector is x (sger.wgsl:38-44),
 * which is this column-major y after its layout swap (sger.mjs:56-64). */
void orc_sger_ld(int64_t m, int64_t n, double alpha, const double *x, int64_t incx,
                 const double *y, int64_t incy, double *A, int64_t lda) {
  if (m == 0 || n == 0 || alpha == 0.0) return;
  for (int64_t j = 0; j < n; ++j) {
    long double yj = y[j * incy];
    if (yj == 0.0L) continue;
    long double t = (long double)alpha * yj;
    for (int64_t i = 0; i < m; ++i)
      A[i + j * lda] = (double)((long double)A[i + j * lda] + (long double)x[i * incx] * t);
  }
}

/* ---- level 2: ssyr / dsyr, ssyr2 / dsyr2 (src/ssyr/ssyr.mjs:17-143,
 * src/ssyr2/ssyr2.mjs:17-184 and their fp64 forms) ------------------------
 * The uplo triangle (1 lower: i >= j, 2 upper: i <= j) of the n x n
 * column-major A <- alpha x x^T + A (syr), or alpha x y^T + alpha y x^T + A
 * (syr2), in long double, in reference BLAS's column order, which the
 * reference's tests hold it to through stdlib (tests/ssyr/src/test.ssyr.js:
 * 111-128, 165-230; test.ssyr2.js:142-161, 202-283): n == 0 or alpha == 0
 * leave A untouched (vectors unread); column j is skipped when x[j] (syr2:
 * x[j] and y[j]) is zero; otherwise A(i, j) += x[i] (alpha x[j]) (syr2:
 * + x[i] (alpha y[j]) + y[i] (alpha x[j])) over the triangle's rows. The
 * other triangle is never touched. In the reference's row-major frame the
 * skipped index is the row (ssyr.wgsl:38-44), this column after its uplo
 * flip (ssyr.mjs:68-71). */
void orc_ssyr2_ld(int uplo, int64_t n, double alpha, const double *x, int64_t incx,
                  const double *y, int64_t incy, int two, double *A, int64_t lda) {
  if (n == 0 || alpha == 0.0) return;
  for (int64_t j = 0; j < n; ++j) {
    long double xj = x[j * incx], yj = two ? y[j * incy] : xj;
    if (xj == 0.0L && (!two || yj == 0.0L)) continue;
    long double t1 = (long double)alpha * yj, t2 = (long double)alpha * xj;
    int64_t lo = uplo == 1 ? j : 0, hi = uplo == 1 ? n : j + 1;
    for (int64_t i = lo; i < hi; ++i) {
      long double v = (long double)A[i + j * lda] + (long double)x[i * incx] * t1;
      if (two) v += (long double)y[i * incy] * t2;
      A[i + j * lda] = (double)v;
    }
  }
}

/* ---- level 2: ssymv / dsymv (src/ssymv/ssymv.mjs:17-216,
 * src/dsymv/dsymv.mjs) ----------------------------------------------------
 * y <- alpha S x + beta y, S the n x n symmetric matrix whose uplo triangle
 * (1 lower, 2 upper) the column-major A holds, in long double, with
 * reference BLAS's rules, which the reference's tests hold it to through
 * stdlib (tests/ssymv/src/test.ssymv.js:147-171, 258-297): n == 0, or
 * alpha == 0 with beta == 1, leave y untouched; alpha == 0 reads neither A
 * nor x; beta == 0 never reads y; every term is taken (no zero skipping).
 * absdot (may be NULL, length n) gets sum_j |S(i, j) x(j)|. */
void orc_ssymv_ld(int uplo, int64_t n, double alpha, const double *A, int64_t lda,
                  const double *x, int64_t incx, double beta, double *y, int64_t incy,
                  double *absdot) {
  if (absdot)
    for (int64_t i = 0; i < n; ++i) absdot[i] = 0.0;
  if (n == 0 || (alpha == 0.0 && beta == 1.0)) return;
  for (int64_t i = 0; i < n; ++i) {
    long double s = 0, a = 0;
    if (alpha != 0.0) {
      for (int64_t j = 0; j < n; ++j) {
        int stored = uplo == 1 ? i >= j : i <= j;
        long double sij = stored ? A[i + j * lda] : A[j + i * lda];
        long double t = sij * (long double)x[j * incx];
        s += t;
        a += fabsl(t);
      }
    }
    long double v = (long double)alpha * s;
    if (beta != 0.0) v += (long double)beta * y[i * incy];
    y[i * incy] = (double)v;
    if (absdot) absdot[i] = (double)a;
  }
}

/* ---- level 2: strmv / dtrmv (src/strmv/strmv.mjs:20-259,
 * src/dtrmv/dtrmv.mjs:24-355) ----------------------------------------------------
 * y <- op(T) x out of place, T the n x n triangle (uplo 1 lower, 2 upper) of
 * the column-major A, op(T) = T (trans 0) or T^T (trans 1), the diagonal
 * taken as 1 when unit (its stored value never read), in long double. The
 * column form (trans 0 here, the reference's row-major transposed kernel,
 * src/shaders/strmv_t.wgsl:44-55) skips a column whose x entry is +-0, so
 * 0 * Inf / NaN of that column never happens; the dot form (trans 1, the
 * row kernel src/shaders/strmv.wgsl:35-47) takes every term. y is written,
 * never read (only its strided slots). absdot (may be NULL, length n) gets
 * sum_j |op(T)(i, j) x(j)| over the terms taken. */
void orc_strmv_ld(int uplo, int trans, int unit, int64_t n, const double *A, int64_t lda,
                  const double *x, int64_t incx, double *y, int64_t incy, double *absdot) {
  for (int64_t i = 0; i < n; ++i) {
    long double s = 0, a = 0;
    for (int64_t j = 0; j < n; ++j) {
      /* element (r, c) of T read for op(T)(i, j) */
      int64_t r = trans ? j : i, c = trans ? i : j;
      int stored = uplo == 1 ? r >= c : r <= c;
      if (!stored) continue;
      double xj = x[j * incx];
      if (!trans && xj == 0.0) continue;
      long double t = (unit && r == c ? 1.0L : (long double)A[r + c * lda]) * (long double)xj;
      s += t;
      a += fabsl(t);
    }
    y[i * incy] = (double)s;
    if (absdot) absdot[i] = (double)a;
  }
}
