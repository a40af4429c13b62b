// Internal declarations shared by the libwgblas_hip translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/wgblas_hip.h"

struct wgb_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  hipEvent_t ev_start = nullptr;
  hipEvent_t ev_stop = nullptr;
  bool timing = false;
  bool timed_once = false;
  float last_ms = 0.0f;
  int num_cus = 0;
  // Device scratch for the two-pass reductions: per-block partials followed
  // by a result slot. Stream order makes reuse across calls safe.
  void *scratch = nullptr;
  size_t scratch_bytes = 0;
  // GEMM split-k workspace: partial tiles of the launch's last, partly
  // filled round (grown on demand, reused in stream order).
  void *gemm_ws = nullptr;
  size_t gemm_ws_bytes = 0;
  // Level-3 operand workspace: ssymm's symmetrized A, strmm's masked A and
  // its copy of B (grown on demand, reused in stream order).
  void *op_ws = nullptr;
  size_t op_ws_bytes = 0;
  // Pinned host slot the host-result reductions copy their scalar into.
  void *host_result = nullptr;
  char name[256] = {0};
  char arch[64] = {0};
};

namespace wgb {

// Records `msg` as the calling thread's last error and returns `status`.
int fail(int status, const std::string &msg);
int fail_hip(hipError_t err, const char *what);

// Makes ctx's device current; every entry point calls it first.
int enter(wgb_ctx *ctx);

// A pointer's 16-byte alignment (vector loads and stores).
inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Brackets a routine's kernels with the context's timing events.
void timing_begin(wgb_ctx *ctx);
void timing_end(wgb_ctx *ctx);

// Largest number of first-pass blocks a reduction may use; the scratch
// buffer is sized for this many 32-byte partials plus the result slot.
constexpr int kMaxReduceBlocks = 4096;
constexpr size_t kScratchBytes = (size_t)kMaxReduceBlocks * 32 + 256;  // 32-byte partial slots + result

// Grows the context's operand workspace (ctx->op_ws) to at least `bytes`;
// the stream is drained first, since an earlier launch may still read it.
// Shared by the level-2 and level-3 routines (one stream orders them).
int ensure_op_workspace(wgb_ctx *ctx, size_t bytes);

// GEMM k-band: which operand is triangular (zero outside its triangle).
enum { kBandNone = 0, kBandALower = 1, kBandAUpper = 2, kBandBLower = 3, kBandBUpper = 4 };
// Order of the diagonal blocks a banded GEMM reads from a side copy
// (gemm_side_*; trmm's copy of its triangle's diagonal blocks).
constexpr int kSideBlock = 128;

// One fp32 GEMM on ctx's stream, C = alpha op(A) op(B) + beta C on the uplo
// part of C (0 = all), without argument checks or timing events.
int gemm_f32(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t m, int64_t n, int64_t k,
             float alpha, const float *A, int64_t lda, const float *B, int64_t ldb, float beta,
             float *C, int64_t ldc, int band);
// The same in fp64.
int gemm_f64(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t m, int64_t n, int64_t k,
             double alpha, const double *A, int64_t lda, const double *B, int64_t ldb,
             double beta, double *C, int64_t ldc, int band);
// C = alpha op(A) op(B) (beta = 0, full C) with one operand banded (band):
// that operand's diagonal kSideBlock x kSideBlock blocks are read from
// `side`, a matrix at the same leading dimension (only those blocks need to
// hold anything), the rest of it in place. trmm's product.
int gemm_side_f32(wgb_ctx *ctx, int transA, int transB, int64_t m, int64_t n, int64_t k, float alpha,
                  const float *A, int64_t lda, const float *B, int64_t ldb, float *C, int64_t ldc,
                  int band, const float *side);
int gemm_side_f64(wgb_ctx *ctx, int transA, int transB, int64_t m, int64_t n, int64_t k, double alpha,
                  const double *A, int64_t lda, const double *B, int64_t ldb, double *C, int64_t ldc,
                  int band, const double *side);
// C = alpha (op(A) op(B) + op(A2) op(B2)) + beta C on the uplo part of C,
// the second pair at the first pair's leading dimensions and transposes:
// one launch over both k ranges where the kernels allow it (ssyr2k /
// dsyr2k), else two.
int gemm2_f32(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t m, int64_t n, int64_t k,
              float alpha, const float *A, const float *A2, int64_t lda, const float *B,
              const float *B2, int64_t ldb, float beta, float *C, int64_t ldc);
int gemm2_f64(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t m, int64_t n, int64_t k,
              double alpha, const double *A, const double *A2, int64_t lda, const double *B,
              const double *B2, int64_t ldb, double beta, double *C, int64_t ldc);
// wgb_sgemm_noalloc's fixed per-GPU split-k workspace (noalloc.hip): its
// size, and its device address on ctx's device (current on entry), looked
// up on the first call for that device.
constexpr size_t kNoallocWsBytes = (size_t)32 << 20;
int noalloc_workspace(wgb_ctx *ctx, void **ptr);
// The GEMM entry points' argument checks.
int check_gemm(int uplo, bool want_uplo, int transA, int transB, int64_t m, int64_t n, int64_t k,
               const void *A, int64_t lda, const void *B, int64_t ldb, const void *C,
               int64_t ldc);

}  // namespace wgb

#define WGB_CHECK_HIP(expr)                               \
  do {                                                    \
    hipError_t _e = (expr);                               \
    if (_e != hipSuccess) return wgb::fail_hip(_e, #expr); \
  } while (0)

#define WGB_CHECK_LAUNCH(what)                                  \
  do {                                                          \
    hipError_t _e = hipGetLastError();                          \
    if (_e != hipSuccess) return wgb::fail_hip(_e, what);       \
  } while (0)
