// Vendor-library twin of bench.py's workloads on one MI355X: the same
// configurations and the same seeded inputs (drawn with this library's
// device fills), computed by rocBLAS, for context next to wgblas_amd's own
// numbers. It plays the role of wgblas's cuBLAS twins
// (benchmarks/<routine>/cuda/<routine>.c): a vendor baseline on the same
// hardware, not a parity check.
//
//   vendor_twin [workload ...]     (no argument: every workload)
//
// One JSON line per workload: the routine, its shape, the median of the
// per-call durations (HIP events on the stream rocBLAS runs on), and
// TFLOP/s or GB/s with the same flop / byte counts bench.py uses.
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "wgblas_hip.h"

namespace {

#define HIP_OK(expr)                                                          \
  do {                                                                        \
    hipError_t e_ = (expr);                                                   \
    if (e_ != hipSuccess) {                                                   \
      std::fprintf(stderr, "%s: %s\n", #expr, hipGetErrorString(e_));         \
      std::exit(1);                                                           \
    }                                                                         \
  } while (0)
#define RB_OK(expr)                                                           \
  do {                                                                        \
    rocblas_status s_ = (expr);                                               \
    if (s_ != rocblas_status_success) {                                       \
      std::fprintf(stderr, "%s: %s\n", #expr, rocblas_status_to_string(s_)); \
      std::exit(1);                                                           \
    }                                                                         \
  } while (0)
#define WGB_OK_(expr)                                                         \
  do {                                                                        \
    if ((expr) != WGB_OK) {                                                   \
      std::fprintf(stderr, "%s: %s\n", #expr, wgb_last_error());              \
      std::exit(1);                                                           \
    }                                                                         \
  } while (0)

struct Twin {
  wgb_ctx *ctx = nullptr;
  hipStream_t stream = nullptr;
  rocblas_handle h = nullptr;
  hipEvent_t a = nullptr, b = nullptr;
  std::vector<void *> bufs;

  float *f32(int64_t n, uint32_t seed, double lo = -1.0, double hi = 1.0) {
    void *p = nullptr;
    WGB_OK_(wgb_malloc(ctx, (size_t)std::max<int64_t>(n, 1) * 4, &p));
    WGB_OK_(wgb_fill_uniform_f32(ctx, (float *)p, n, lo, hi, seed));
    bufs.push_back(p);
    return (float *)p;
  }
  double *f64(int64_t n, uint32_t seed) {
    void *p = nullptr;
    WGB_OK_(wgb_malloc(ctx, (size_t)std::max<int64_t>(n, 1) * 8, &p));
    WGB_OK_(wgb_fill_uniform_f64(ctx, (double *)p, n, -1.0, 1.0, seed));
    bufs.push_back(p);
    return (double *)p;
  }
  void release() {
    WGB_OK_(wgb_synchronize(ctx));
    for (void *p : bufs) WGB_OK_(wgb_free(ctx, p));
    bufs.clear();
  }
  // median of `iters` per-call durations after at least `warmup` untimed
  // calls and ~30 ms of them (bench.py's warm_up: the clocks take some tens
  // of milliseconds of load to settle after the set-up between workloads);
  // `before` (untimed) runs ahead of every call
  double median_ms(const std::function<void()> &f, int warmup, int iters,
                   const std::function<void()> &before = nullptr) {
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < 400; ++i) {
      if (before) before();
      f();
      if (i + 1 >= warmup && (i + 1) % 4 == 0) {
        HIP_OK(hipStreamSynchronize(stream));
        if (std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() >= 30.0)
          break;
      }
    }
    std::vector<float> t;
    for (int i = 0; i < iters; ++i) {
      if (before) before();
      HIP_OK(hipEventRecord(a, stream));
      f();
      HIP_OK(hipEventRecord(b, stream));
      HIP_OK(hipEventSynchronize(b));
      float ms = 0;
      HIP_OK(hipEventElapsedTime(&ms, a, b));
      t.push_back(ms);
    }
    std::sort(t.begin(), t.end());
    return t[t.size() / 2];
  }
};

void emit(const char *name, const char *shape, double ms, double work, const char *unit) {
  const double rate = std::strcmp(unit, "TFLOP/s") == 0 ? work / ms / 1e9 : work / ms / 1e6;
  std::printf("{\"workload\": \"%s\", \"library\": \"rocBLAS\", \"shape\": \"%s\", \"ms\": %.5f, "
              "\"%s\": %.3f}\n",
              name, shape, ms, unit, rate);
  std::fflush(stdout);
}

rocblas_operation op(char t) { return t == 'T' ? rocblas_operation_transpose : rocblas_operation_none; }

void run_gemm8192(Twin &w) {
  const int n = 8192;
  float *A = w.f32((int64_t)3 * n * n, 2);  // A, B, C consecutive in one stream (config 3)
  float *B = A + (int64_t)n * n, *C = B + (int64_t)n * n;
  const float alpha = 1.5f, beta = 0.5f;
  for (const char *tt : {"NN", "NT", "TN", "TT"}) {
    const double ms = w.median_ms(
        [&] { RB_OK(rocblas_sgemm(w.h, op(tt[0]), op(tt[1]), n, n, n, &alpha, A, n, B, n, &beta, C, n)); },
        3, 10);
    char name[32];
    std::snprintf(name, sizeof name, "sgemm_8192_%s", tt);
    emit(name, "8192^3 alpha 1.5 beta 0.5", ms, 2.0 * n * n * (double)n, "TFLOP/s");
  }
  w.release();
}

void run_gemm512(Twin &w) {
  const int n = 512;
  float *A = w.f32((int64_t)3 * n * n, 0);
  float *B = A + n * n, *C = B + n * n;
  const float one = 1.f, zero = 0.f;
  const double ms = w.median_ms(
      [&] { RB_OK(rocblas_sgemm(w.h, op('N'), op('N'), n, n, n, &one, A, n, B, n, &zero, C, n)); }, 10, 50);
  emit("sgemm_512", "512^3 NN alpha 1 beta 0", ms, 2.0 * n * n * (double)n, "TFLOP/s");
  w.release();
}

void run_ragged(Twin &w) {
  const int m = 8191, n = 8193, k = 4097;
  auto ld = [](int r) { return (r + 63) / 64 * 64 + 1; };
  const int lda = ld(m), ldb = ld(k), ldc = ld(m);
  float *A = w.f32((int64_t)lda * k + (int64_t)ldb * n + (int64_t)ldc * n, 2);
  float *B = A + (int64_t)lda * k, *C = B + (int64_t)ldb * n;
  const float alpha = 1.5f, beta = 0.5f;
  const double ms = w.median_ms(
      [&] { RB_OK(rocblas_sgemm(w.h, op('N'), op('N'), m, n, k, &alpha, A, lda, B, ldb, &beta, C, ldc)); },
      3, 10);
  emit("sgemm_ragged", "8191x8193x4097 NN, ld = 1 mod 64", ms, 2.0 * m * n * (double)k, "TFLOP/s");
  w.release();
}

void run_dgemm(Twin &w) {
  const int n = 4096;
  double *A = w.f64((int64_t)3 * n * n, 3);
  double *B = A + (int64_t)n * n, *C = B + (int64_t)n * n;
  const double one = 1.0;
  const double ms = w.median_ms(
      [&] { RB_OK(rocblas_dgemm(w.h, op('N'), op('T'), n, n, n, &one, A, n, B, n, &one, C, n)); }, 3, 10);
  emit("dgemm_4096", "4096^3 NT alpha 1 beta 1", ms, 2.0 * n * n * (double)n, "TFLOP/s");
  w.release();
}

void run_syrk_family(Twin &w) {
  const int n = 8192, k = 4096;
  float *A = w.f32((int64_t)n * k, 4), *B = w.f32((int64_t)n * k, 6), *C = w.f32((int64_t)n * n, 5);
  const float one = 1.f, quarter = 0.25f;
  double ms = w.median_ms(
      [&] {
        RB_OK(rocblas_ssyrk(w.h, rocblas_fill_lower, op('N'), n, k, &one, A, n, &quarter, C, n));
      },
      2, 10);
  emit("ssyrk_8192x4096", "lower N n 8192 k 4096 beta 0.25", ms, (double)n * (n + 1) * k, "TFLOP/s");
  ms = w.median_ms(
      [&] {
        RB_OK(rocblas_sgemmt(w.h, rocblas_fill_lower, op('N'), op('T'), n, k, &one, A, n, A, n, &quarter,
                             C, n));
      },
      2, 10);
  emit("sgemmtr_8192x4096", "lower A A^T n 8192 k 4096 beta 0.25", ms, (double)n * (n + 1) * k,
       "TFLOP/s");
  ms = w.median_ms(
      [&] {
        RB_OK(rocblas_ssyr2k(w.h, rocblas_fill_lower, op('N'), n, k, &one, A, n, B, n, &quarter, C, n));
      },
      2, 10);
  emit("ssyr2k_8192x4096", "lower N n 8192 k 4096 beta 0.25", ms, 2.0 * n * (n + 1) * (double)k,
       "TFLOP/s");
  w.release();
}

void run_level3(Twin &w) {
  const int n = 8192;
  float *A = w.f32((int64_t)n * n, 7), *B = w.f32((int64_t)n * n, 8), *C = w.f32((int64_t)n * n, 9);
  const float one = 1.f, half = 0.5f;
  double ms = w.median_ms(
      [&] {
        RB_OK(rocblas_ssymm(w.h, rocblas_side_left, rocblas_fill_lower, n, n, &one, A, n, B, n, &half, C,
                            n));
      },
      2, 10);
  emit("ssymm_8192", "left lower 8192^2", ms, 2.0 * n * n * (double)n + 2.0 * n * n, "TFLOP/s");
  // rocBLAS's strmm writes C (out of place); B and C distinct
  ms = w.median_ms(
      [&] {
        RB_OK(rocblas_strmm(w.h, rocblas_side_left, rocblas_fill_lower, op('N'), rocblas_diagonal_non_unit,
                            n, n, &one, A, n, B, n, C, n));
      },
      2, 10);
  emit("strmm_8192", "left lower N non-unit 8192^2 (TFLOP/s of the triangle, n^3)", ms,
       (double)n * n * n, "TFLOP/s");
  w.release();
  for (int order : {4096, 8192}) {
    // a well-conditioned lower triangle: off-diagonals in [-1/n, 1/n),
    // diagonal 2 (bench.py's strsm input); B refilled before each solve
    float *T = w.f32((int64_t)order * order, 10, -1.0 / order, 1.0 / order);
    std::vector<float> two(1, 2.f);
    for (int i = 0; i < order; ++i)
      WGB_OK_(wgb_memcpy_h2d(w.ctx, T + (int64_t)i * order + i, two.data(), 4));
    float *X = w.f32((int64_t)order * order, 11);
    const double ms2 = w.median_ms(
        [&] {
          RB_OK(rocblas_strsm(w.h, rocblas_side_left, rocblas_fill_lower, op('N'), rocblas_diagonal_non_unit,
                              order, order, &one, T, order, X, order));
        },
        1, 5, [&] { WGB_OK_(wgb_fill_uniform_f32(w.ctx, X, (int64_t)order * order, -1.0, 1.0, 11)); });
    char name[32];
    std::snprintf(name, sizeof name, "strsm_%d", order);
    emit(name, "left lower N non-unit, n x n right-hand sides", ms2, (double)order * order * order,
         "TFLOP/s");
    w.release();
  }
}

// dsyr2k (k = n), dsymm and dtrmm at order 4096: bench.py's fp64 level-3
// components (left, lower, no transpose, alpha 1, beta 0)
void run_level3_f64(Twin &w) {
  const int n = 4096;
  double *A = w.f64((int64_t)n * n, 7), *B = w.f64((int64_t)n * n, 8), *C = w.f64((int64_t)n * n, 9);
  const double one = 1.0, zero = 0.0;
  double ms = w.median_ms(
      [&] {
        RB_OK(rocblas_dsyr2k(w.h, rocblas_fill_lower, op('N'), n, n, &one, A, n, B, n, &zero, C, n));
      },
      2, 10);
  emit("dsyr2k_4096", "lower N n = k = 4096 beta 0", ms, 2.0 * n * (n + 1) * (double)n, "TFLOP/s");
  ms = w.median_ms(
      [&] {
        RB_OK(rocblas_dsymm(w.h, rocblas_side_left, rocblas_fill_lower, n, n, &one, A, n, B, n, &zero, C,
                            n));
      },
      2, 10);
  emit("dsymm_4096", "left lower 4096^2 beta 0", ms, 2.0 * n * n * (double)n + 2.0 * n * n, "TFLOP/s");
  // out of place, as strmm above: B and C distinct
  ms = w.median_ms(
      [&] {
        RB_OK(rocblas_dtrmm(w.h, rocblas_side_left, rocblas_fill_lower, op('N'), rocblas_diagonal_non_unit,
                            n, n, &one, A, n, B, n, C, n));
      },
      2, 10);
  emit("dtrmm_4096", "left lower N non-unit 4096^2 (TFLOP/s of the triangle, n^3)", ms,
       (double)n * n * n, "TFLOP/s");
  w.release();
}

void run_gemv(Twin &w) {
  const int n = 16384;
  float *A = w.f32((int64_t)n * n, 12), *x = w.f32(n, 13), *y = w.f32(n, 14);
  const float one = 1.f, half = 0.5f;
  for (char t : {'N', 'T'}) {
    const double ms = w.median_ms(
        [&] { RB_OK(rocblas_sgemv(w.h, op(t), n, n, &one, A, n, x, 1, &half, y, 1)); }, 5, 20);
    char name[32];
    std::snprintf(name, sizeof name, "sgemv_%c_16384", t);
    emit(name, "16384^2, 1 GiB of A", ms, 4.0 * ((double)n * n + 3.0 * n), "GB/s");
  }
  w.release();
  double *Ad = w.f64((int64_t)n * n, 12), *xd = w.f64(n, 13), *yd = w.f64(n, 14);
  const double oned = 1.0, halfd = 0.5;
  for (char t : {'N', 'T'}) {
    const double ms = w.median_ms(
        [&] { RB_OK(rocblas_dgemv(w.h, op(t), n, n, &oned, Ad, n, xd, 1, &halfd, yd, 1)); }, 5, 20);
    char name[32];
    std::snprintf(name, sizeof name, "dgemv_%c_16384", t);
    emit(name, "16384^2, 2 GiB of A", ms, 8.0 * ((double)n * n + 3.0 * n), "GB/s");
  }
  w.release();
  // sger / dger on the same shape (A read and written), alpha 1e-3
  {
    float *A = w.f32((int64_t)n * n, 15), *x = w.f32(n, 16), *y = w.f32(n, 17);
    const float a = 1e-3f;
    const double ms = w.median_ms([&] { RB_OK(rocblas_sger(w.h, n, n, &a, x, 1, y, 1, A, n)); }, 5, 20);
    emit("sger_16384", "16384^2, A read and written", ms, 4.0 * (2.0 * n * n + 2.0 * n), "GB/s");
    w.release();
  }
  {
    double *A = w.f64((int64_t)n * n, 15), *x = w.f64(n, 16), *y = w.f64(n, 17);
    const double a = 1e-3;
    const double ms = w.median_ms([&] { RB_OK(rocblas_dger(w.h, n, n, &a, x, 1, y, 1, A, n)); }, 5, 20);
    emit("dger_16384", "16384^2, A read and written", ms, 8.0 * (2.0 * n * n + 2.0 * n), "GB/s");
    w.release();
  }
  // ssyr / ssyr2 / dsyr / dsyr2 (lower): the triangle read and written
  {
    float *A = w.f32((int64_t)n * n, 15), *x = w.f32(n, 16), *y = w.f32(n, 17);
    const float a = 1e-3f;
    double ms = w.median_ms(
        [&] { RB_OK(rocblas_ssyr(w.h, rocblas_fill_lower, n, &a, x, 1, A, n)); }, 5, 20);
    emit("ssyr_16384", "lower 16384, triangle read and written", ms,
         4.0 * ((double)n * (n + 1) + n), "GB/s");
    ms = w.median_ms(
        [&] { RB_OK(rocblas_ssyr2(w.h, rocblas_fill_lower, n, &a, x, 1, y, 1, A, n)); }, 5, 20);
    emit("ssyr2_16384", "lower 16384, triangle read and written", ms,
         4.0 * ((double)n * (n + 1) + 2.0 * n), "GB/s");
    w.release();
  }
  {
    double *A = w.f64((int64_t)n * n, 15), *x = w.f64(n, 16), *y = w.f64(n, 17);
    const double a = 1e-3;
    double ms = w.median_ms(
        [&] { RB_OK(rocblas_dsyr(w.h, rocblas_fill_lower, n, &a, x, 1, A, n)); }, 5, 20);
    emit("dsyr_16384", "lower 16384, triangle read and written", ms,
         8.0 * ((double)n * (n + 1) + n), "GB/s");
    ms = w.median_ms(
        [&] { RB_OK(rocblas_dsyr2(w.h, rocblas_fill_lower, n, &a, x, 1, y, 1, A, n)); }, 5, 20);
    emit("dsyr2_16384", "lower 16384, triangle read and written", ms,
         8.0 * ((double)n * (n + 1) + 2.0 * n), "GB/s");
    w.release();
  }
  // ssymv / dsymv (lower): the triangle read once
  {
    float *A = w.f32((int64_t)n * n, 18), *x = w.f32(n, 19), *y = w.f32(n, 20);
    const float one = 1.f, half = 0.5f;
    const double ms = w.median_ms(
        [&] { RB_OK(rocblas_ssymv(w.h, rocblas_fill_lower, n, &one, A, n, x, 1, &half, y, 1)); }, 5, 20);
    emit("ssymv_16384", "lower 16384, triangle read once", ms, 4.0 * ((double)n * (n + 1) / 2 + 3.0 * n),
         "GB/s");
    w.release();
  }
  {
    double *A = w.f64((int64_t)n * n, 18), *x = w.f64(n, 19), *y = w.f64(n, 20);
    const double one = 1.0, half = 0.5;
    const double ms = w.median_ms(
        [&] { RB_OK(rocblas_dsymv(w.h, rocblas_fill_lower, n, &one, A, n, x, 1, &half, y, 1)); }, 5, 20);
    emit("dsymv_16384", "lower 16384, triangle read once", ms, 8.0 * ((double)n * (n + 1) / 2 + 3.0 * n),
         "GB/s");
    w.release();
  }
  // strmv / dtrmv (lower, both forms; rocBLAS's is in place, x <- op(T) x,
  // the same bytes): the triangle read once, x read and written
  for (int t = 0; t < 2; ++t) {
    const rocblas_operation op = t ? rocblas_operation_transpose : rocblas_operation_none;
    {
      float *A = w.f32((int64_t)n * n, 21), *x = w.f32(n, 22);
      const double ms = w.median_ms(
          [&] { RB_OK(rocblas_strmv(w.h, rocblas_fill_lower, op, rocblas_diagonal_non_unit, n, A, n, x, 1)); },
          5, 20);
      emit(t ? "strmv_T_16384" : "strmv_N_16384", "lower 16384, triangle read once", ms,
           4.0 * ((double)n * (n + 1) / 2 + 2.0 * n), "GB/s");
      w.release();
    }
    {
      double *A = w.f64((int64_t)n * n, 21), *x = w.f64(n, 22);
      const double ms = w.median_ms(
          [&] { RB_OK(rocblas_dtrmv(w.h, rocblas_fill_lower, op, rocblas_diagonal_non_unit, n, A, n, x, 1)); },
          5, 20);
      emit(t ? "dtrmv_T_16384" : "dtrmv_N_16384", "lower 16384, triangle read once", ms,
           8.0 * ((double)n * (n + 1) / 2 + 2.0 * n), "GB/s");
      w.release();
    }
  }
}

void run_level1(Twin &w) {
  RB_OK(rocblas_set_pointer_mode(w.h, rocblas_pointer_mode_device));
  const int n = 1 << 28;
  float *x = w.f32(n, 1), *y = w.f32(n, 2), *r = w.f32(4, 0);
  rocblas_int *ri = nullptr;
  WGB_OK_(wgb_malloc(w.ctx, 8, (void **)&ri));
  w.bufs.push_back(ri);
  const double bytes1 = 4.0 * n;
  emit("sdot_2^28", "n 2^28", w.median_ms([&] { RB_OK(rocblas_sdot(w.h, n, x, 1, y, 1, r)); }, 5, 50),
       2 * bytes1, "GB/s");
  emit("sasum_2^28", "n 2^28", w.median_ms([&] { RB_OK(rocblas_sasum(w.h, n, x, 1, r)); }, 5, 50), bytes1,
       "GB/s");
  emit("snrm2_2^28", "n 2^28", w.median_ms([&] { RB_OK(rocblas_snrm2(w.h, n, x, 1, r)); }, 5, 50), bytes1,
       "GB/s");
  emit("isamax_2^28", "n 2^28", w.median_ms([&] { RB_OK(rocblas_isamax(w.h, n, x, 1, ri)); }, 5, 50),
       bytes1, "GB/s");
  w.release();
  const int nd = 1 << 27;
  double *dx = w.f64(nd, 1), *dy = w.f64(nd, 2), *dr = w.f64(4, 0);
  WGB_OK_(wgb_malloc(w.ctx, 8, (void **)&ri));
  w.bufs.push_back(ri);
  const double bytesd = 8.0 * nd;
  emit("ddot_2^27", "n 2^27", w.median_ms([&] { RB_OK(rocblas_ddot(w.h, nd, dx, 1, dy, 1, dr)); }, 5, 50),
       2 * bytesd, "GB/s");
  emit("dasum_2^27", "n 2^27", w.median_ms([&] { RB_OK(rocblas_dasum(w.h, nd, dx, 1, dr)); }, 5, 50),
       bytesd, "GB/s");
  emit("dnrm2_2^27", "n 2^27", w.median_ms([&] { RB_OK(rocblas_dnrm2(w.h, nd, dx, 1, dr)); }, 5, 50),
       bytesd, "GB/s");
  emit("idamax_2^27", "n 2^27", w.median_ms([&] { RB_OK(rocblas_idamax(w.h, nd, dx, 1, ri)); }, 5, 50),
       bytesd, "GB/s");
  w.release();
  RB_OK(rocblas_set_pointer_mode(w.h, rocblas_pointer_mode_host));
}

}  // namespace

int main(int argc, char **argv) {
  Twin w;
  WGB_OK_(wgb_init(0, &w.ctx));
  w.stream = (hipStream_t)wgb_stream(w.ctx);
  RB_OK(rocblas_create_handle(&w.h));
  RB_OK(rocblas_set_stream(w.h, w.stream));
  HIP_OK(hipEventCreate(&w.a));
  HIP_OK(hipEventCreate(&w.b));
  char ver[128] = {0};
  RB_OK(rocblas_get_version_string(ver, sizeof ver));
  std::fprintf(stderr, "rocBLAS %s\n", ver);
  struct Item {
    const char *name;
    void (*fn)(Twin &);
  } items[] = {{"sgemm_8192", run_gemm8192}, {"sgemm_512", run_gemm512},  {"sgemm_ragged", run_ragged},
               {"dgemm_4096", run_dgemm},    {"syrk", run_syrk_family},    {"level3", run_level3},
               {"level3_f64", run_level3_f64},
               {"sgemv", run_gemv},          {"level1", run_level1}};
  for (const Item &it : items) {
    bool want = argc < 2;
    for (int i = 1; i < argc; ++i) want = want || std::strcmp(argv[i], it.name) == 0;
    if (want) it.fn(w);
  }
  HIP_OK(hipEventDestroy(w.a));
  HIP_OK(hipEventDestroy(w.b));
  RB_OK(rocblas_destroy_handle(w.h));
  WGB_OK_(wgb_destroy(w.ctx));
  return 0;
}
