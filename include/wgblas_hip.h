/*
 * wgblas_hip.h — C ABI of libwgblas_hip, the MI355X (gfx950) implementation
 * of wgblas's data-parallel hot path: the GEMM family (sgemm, sgemmtr, ssyrk,
 * dgemm) and the level-1 reductions (sdot, sasum, snrm2, isamax).
 *
 * Every entry point takes plain pointers and sizes. Matrices are
 * COLUMN-MAJOR (element (i, j) of an ld-strided matrix sits at p[i + j*ld]);
 * the JavaScript shim maps wgblas's row-major/column-major `layout` argument
 * onto this frame. All device pointers must come from wgb_malloc (or any
 * hipMalloc allocation on the context's device). Calls on one context are
 * ordered on that context's single HIP stream.
 *
 * Each routine here replaces the WGSL dispatch path of the reference routine
 * cited beside it (paths relative to the wgblas repository root). The
 * reference does its argument checks in JavaScript; this library repeats the
 * checks that protect memory (sizes, leading dimensions, null pointers) and
 * reports them as WGB_ERR_INVALID_VALUE with a message from wgb_last_error().
 *
 * Return value of every function: WGB_OK (0) or a negative wgb_status.
 */
#ifndef WGBLAS_HIP_H
#define WGBLAS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Version of this interface: raised whenever an entry point's signature or
 * meaning changes (3: wgb_ssyr2k takes a trans flag per operand and
 * wgb_ssymm / wgb_dsymm one for B). A caller compares wgb_abi_version()
 * with the WGB_ABI_VERSION it was built against before its first call. */
#define WGB_ABI_VERSION 3

typedef enum wgb_status {
  WGB_OK = 0,
  WGB_ERR_INVALID_VALUE = -1, /* bad argument (see wgb_last_error) */
  WGB_ERR_HIP = -2,           /* a HIP runtime call failed */
  WGB_ERR_ALLOC = -3,         /* device allocation failed */
  WGB_ERR_NO_DEVICE = -4,     /* no HIP device with that index */
  WGB_ERR_NOT_INITIALIZED = -5
} wgb_status;

/* trans arguments: wgblas's 'no-transpose' / 'transpose' strings. */
enum { WGB_NO_TRANS = 0, WGB_TRANS = 1 };
/* uplo arguments: wgblas's 'lower' / 'upper' strings (column-major frame). */
enum { WGB_LOWER = 1, WGB_UPPER = 2 };
/* side of the symmetric / triangular operand in ssymm, strmm, strsm */
enum { WGB_LEFT = 1, WGB_RIGHT = 2 };
/* diagonal of the triangular operand in strmm, strsm (WGB_UNIT: taken as 1,
 * never read) */
enum { WGB_NON_UNIT = 0, WGB_UNIT = 1 };

typedef struct wgb_ctx wgb_ctx;

/* WGB_ABI_VERSION of the built library (no device work; callable before
 * wgb_init). No counterpart in the reference, whose JavaScript API has no
 * compiled boundary to version. */
int wgb_abi_version(void);

/* ---- device / context ---------------------------------------------------- */

/* Opens HIP device `device` and creates the context's stream.
 * Replaces init() (src/init.mjs:31-108): returns a device handle in place of
 * a GPUDevice. */
int wgb_init(int device, wgb_ctx **out);

/* Waits for the context's work, frees its scratch and stream.
 * Replaces cleanup(device) (src/init.mjs:110-131). */
int wgb_destroy(wgb_ctx *ctx);

/* Writes the device's marketing name and gfx architecture name.
 * Replaces gpuName() (src/init.mjs:133-143). */
int wgb_device_name(wgb_ctx *ctx, char *name, size_t name_len, char *arch,
                    size_t arch_len);

/* Number of visible HIP devices (0 when none). */
int wgb_device_count(int *count);

/* Turns per-call GPU timing on or off. When on, every routine records HIP
 * events around its kernels and wgb_last_time_ms() returns the span.
 * Replaces init({benchmark:true}) + timestamp queries
 * (src/util/benchmark.mjs:14-103, the routines' `gpuTimeMs`). */
int wgb_set_timing(wgb_ctx *ctx, int enabled);
int wgb_last_time_ms(wgb_ctx *ctx, float *ms);

/* Blocks until all work on the context's stream is done. */
int wgb_synchronize(wgb_ctx *ctx);

/* The context's HIP stream (a hipStream_t), for callers that order their own
 * work with the library's. */
void *wgb_stream(wgb_ctx *ctx);

/* Message for the last failure on the calling thread ("" if none). */
const char *wgb_last_error(void);
const char *wgb_status_string(int status);

/* ---- device memory (GpuVector / GpuMatrix residency) ----------------------- */

/* Device allocation of `bytes` (256-byte aligned). Replaces the GPUBuffer
 * that GpuVector.from / GpuMatrix.from create through uploadBuffer
 * (src/classes/GpuVector.mjs:41-74, src/classes/GpuMatrix.mjs:43-140,
 * src/util/buffer.mjs:58-77). */
int wgb_malloc(wgb_ctx *ctx, size_t bytes, void **dptr);
/* Replaces GpuVector/GpuMatrix.destroy() (GpuVector.mjs:102, GpuMatrix.mjs:204). */
int wgb_free(wgb_ctx *ctx, void *dptr);
/* Host -> device copy, ordered on the context's stream and complete on return.
 * Replaces queue.writeBuffer (src/util/buffer.mjs:73-74). */
int wgb_memcpy_h2d(wgb_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Device -> host copy, complete on return. Replaces stageReadback +
 * extractResult (src/util/buffer.mjs:160-185, src/util/result.mjs:18-30). */
int wgb_memcpy_d2h(wgb_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Device -> device copy on the context's stream (asynchronous). */
int wgb_memcpy_d2d(wgb_ctx *ctx, void *dst, const void *src, size_t bytes);

/* ---- seeded synthetic inputs --------------------------------------------- */

/* Fills d_out[0..n) with wgblas's randomFloat32Array(n, low, high, seed)
 * sequence, bit for bit (mulberry32, src/random/random.mjs:4-19), generated
 * on the device. */
int wgb_fill_uniform_f32(wgb_ctx *ctx, float *d_out, int64_t n, double low,
                         double high, uint32_t seed);
/* randomFloat64Array(n, low, high, seed) (src/random/random.mjs:21-26). */
int wgb_fill_uniform_f64(wgb_ctx *ctx, double *d_out, int64_t n, double low,
                         double high, uint32_t seed);
/* normal(0,1) samples, defined by this library (the reference has none):
 * Box-Muller over the same mulberry32(seed) stream. Pair p uses draws
 * u1 = next() (the 2p-th) and u2 = next() (the (2p+1)-th), r = sqrt(-2 ln(1-u1)),
 * t = 2 pi u2; element 2p = r cos t, element 2p+1 = r sin t, in float64,
 * rounded to float32. */
int wgb_fill_normal_f32(wgb_ctx *ctx, float *d_out, int64_t n, uint32_t seed);

/* ---- level 3 ------------------------------------------------------------- */

/* C <- alpha*op(A)*op(B) + beta*C, C m-by-n, op(A) m-by-k, op(B) k-by-n.
 * beta == 0 never reads C; alpha == 0 or k == 0 reads neither A nor B
 * (C <- beta*C). m == 0 or n == 0 is a no-op.
 * Replaces sgemm (src/sgemm/sgemm.mjs:25-269, kernels
 * src/shaders/sgemm_large.wgsl, sgemm_small.wgsl). */
int wgb_sgemm(wgb_ctx *ctx, int transA, int transB, int64_t m, int64_t n,
              int64_t k, float alpha, const float *A, int64_t lda,
              const float *B, int64_t ldb, float beta, float *C, int64_t ldc);

/* Allocation-free sgemm: wgb_sgemm's operation, launches and results (the
 * same bits on the same inputs), with its split-k workspace taken from a
 * fixed 32 MiB device array of the library instead of a buffer grown with
 * hipMalloc; the call makes no hipMalloc, hipFree or other allocation.
 * The first call on each device (not under graph capture) looks the array
 * up, which makes the HIP runtime load its code object and place the array
 * on that device: that one-time load is the only device memory the entry
 * point ever causes to be reserved; every later call allocates nothing.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation). Each GPU holds one copy of the array until the process ends,
 * shared by every call on that GPU and keeping the last call's contents:
 * calls that overlap on one GPU (two contexts' streams, or two host threads)
 * race on it. A problem whose split-k tail would need more than 32 MiB is
 * rejected with WGB_ERR_INVALID_VALUE (on MI355X's 256 CUs no problem does:
 * the tail holds at most one round of 128 x 128 tiles, 32 MiB). */
int wgb_sgemm_noalloc(wgb_ctx *ctx, int transA, int transB, int64_t m,
                      int64_t n, int64_t k, float alpha, const float *A,
                      int64_t lda, const float *B, int64_t ldb, float beta,
                      float *C, int64_t ldc);

/* Same as wgb_sgemm on the uplo triangle of the m-by-n C only
 * (WGB_LOWER: i >= j, WGB_UPPER: i <= j); the other triangle is never read
 * nor written. Replaces sgemmtr (src/sgemmtr/sgemmtr.mjs:25-278). */
int wgb_sgemmtr(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t m,
                int64_t n, int64_t k, float alpha, const float *A, int64_t lda,
                const float *B, int64_t ldb, float beta, float *C,
                int64_t ldc);

/* C <- alpha*op(A)*op(A)^T + beta*C on the uplo triangle of the n-by-n C;
 * op(A) is n-by-k (trans == WGB_NO_TRANS) or A^T for a k-by-n A.
 * Replaces ssyrk (src/ssyrk/ssyrk.mjs:28-244), without its A->B copy. */
int wgb_ssyrk(wgb_ctx *ctx, int uplo, int trans, int64_t n, int64_t k,
              float alpha, const float *A, int64_t lda, float beta, float *C,
              int64_t ldc);

/* Native-FP64 dgemm with wgblas's dgemm contract, including the quick return
 * (alpha == 0 or k == 0) and beta == 1 -> C untouched.
 * Replaces dgemm (src/dgemm/dgemm.mjs:23-318, kernel
 * src/shaders/dgemm_small.wgsl and the double-double library
 * src/shaders/f64/). */
int wgb_dgemm(wgb_ctx *ctx, int transA, int transB, int64_t m, int64_t n,
              int64_t k, double alpha, const double *A, int64_t lda,
              const double *B, int64_t ldb, double beta, double *C,
              int64_t ldc);

/* Native-FP64 dgemmtr: dgemm's operation on the uplo triangle of the m-by-n
 * C only, with dgemm's quick return. Replaces dgemmtr
 * (src/dgemmtr/dgemmtr.mjs:25-328, which runs dgemm_small with its triangle
 * mask). */
int wgb_dgemmtr(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t m,
                int64_t n, int64_t k, double alpha, const double *A,
                int64_t lda, const double *B, int64_t ldb, double beta,
                double *C, int64_t ldc);

/* Native-FP64 dsyrk: C <- alpha*op(A)*op(A)^T + beta*C on the uplo triangle
 * of the n-by-n C, with dgemm's quick return; A is read once for both
 * operands. Replaces dsyrk (src/dsyrk/dsyrk.mjs:28-305, which copies A into
 * a second buffer). */
int wgb_dsyrk(wgb_ctx *ctx, int uplo, int trans, int64_t n, int64_t k,
              double alpha, const double *A, int64_t lda, double beta,
              double *C, int64_t ldc);

/* C <- alpha*op(A)*op(B)^T + alpha*op(B)*op(A)^T + beta*C on the uplo
 * triangle of the n-by-n C; op(X) is n-by-k (trans flag WGB_NO_TRANS) or X^T
 * for a k-by-n X. wgblas has one trans for both operands; a flag per operand
 * takes its GpuMatrix operands of different storage orders in one call.
 * Two triangle GEMM launches, the second with beta = 1, as wgblas runs it,
 * timed as one span; alpha == 0 or k == 0 is C <- beta*C on the triangle
 * without reading A or B.
 * Replaces ssyr2k (src/ssyr2k/ssyr2k.mjs:27-301). */
int wgb_ssyr2k(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t n,
               int64_t k, float alpha, const float *A, int64_t lda,
               const float *B, int64_t ldb, float beta, float *C, int64_t ldc);

/* Native-FP64 dsyr2k: wgb_ssyr2k's operation in fp64, with reference BLAS's
 * quick return (alpha == 0 or k == 0 with beta == 1 leaves C,
 * src/dsyr2k/dsyr2k.mjs:172-174). Replaces dsyr2k
 * (src/dsyr2k/dsyr2k.mjs:24-331, two dgemm_small passes with its triangle
 * mask in double-double). */
int wgb_dsyr2k(wgb_ctx *ctx, int uplo, int transA, int transB, int64_t n,
               int64_t k, double alpha, const double *A, int64_t lda,
               const double *B, int64_t ldb, double beta, double *C,
               int64_t ldc);

/* C <- alpha*A*op(B) + beta*C (side WGB_LEFT, A m-by-m) or
 * alpha*op(B)*A + beta*C (WGB_RIGHT, A n-by-n); A symmetric, only its uplo
 * triangle is read. C and op(B) are m-by-n: B is stored m-by-n (transB ==
 * WGB_NO_TRANS) or n-by-m (WGB_TRANS, wgblas's B and C of different storage
 * orders, src/ssymm/ssymm.mjs:85-87, 149-163). alpha == 0 reads neither A
 * nor B. Replaces ssymm (src/ssymm/ssymm.mjs:30-318: symmetrize.wgsl, then
 * sgemm). */
int wgb_ssymm(wgb_ctx *ctx, int side, int uplo, int transB, int64_t m,
              int64_t n, float alpha, const float *A, int64_t lda,
              const float *B, int64_t ldb, float beta, float *C, int64_t ldc);

/* Native-FP64 dsymm: wgb_ssymm's operation in fp64, with reference BLAS's
 * quick return (alpha == 0 with beta == 1 leaves C,
 * src/dsymm/dsymm.mjs:143-145). Replaces dsymm (src/dsymm/dsymm.mjs:26-381:
 * symmetrize.wgsl on both halves, then dgemm_small in double-double). */
int wgb_dsymm(wgb_ctx *ctx, int side, int uplo, int transB, int64_t m,
              int64_t n, double alpha, const double *A, int64_t lda,
              const double *B, int64_t ldb, double beta, double *C,
              int64_t ldc);

/* B <- alpha*op(A)*B (WGB_LEFT, A m-by-m) or alpha*B*op(A) (WGB_RIGHT,
 * A n-by-n); A triangular (uplo triangle read; diag WGB_UNIT takes its
 * diagonal as 1 without reading it). B is m-by-n, overwritten in place;
 * its ld padding is untouched. alpha == 0 sets B to zero without reading A
 * or B. Replaces strmm (src/strmm/strmm.mjs:30-344: triangularize.wgsl,
 * then sgemm with its k band). */
int wgb_strmm(wgb_ctx *ctx, int side, int uplo, int transA, int diag,
              int64_t m, int64_t n, float alpha, const float *A, int64_t lda,
              float *B, int64_t ldb);

/* Native-FP64 dtrmm: wgb_strmm's operation in fp64 (alpha == 0 sets B to
 * zero); like wgb_strmm, the GEMM runs only the k-tiles the triangle
 * reaches (wgblas's dtrmm multiplies the whole zero-filled copy). Replaces
 * dtrmm (src/dtrmm/dtrmm.mjs:28-400:
 * triangularize.wgsl on both halves, then dgemm_small). */
int wgb_dtrmm(wgb_ctx *ctx, int side, int uplo, int transA, int diag,
              int64_t m, int64_t n, double alpha, const double *A, int64_t lda,
              double *B, int64_t ldb);

/* Solves op(A)*X = alpha*B (WGB_LEFT, A m-by-m) or X*op(A) = alpha*B
 * (WGB_RIGHT, A n-by-n) for X, overwriting the m-by-n B; A triangular as in
 * wgb_strmm. Substitution on diagonal blocks of order <= 256 (inside 16-row
 * sub-blocks, MFMA updates between them), GEMM updates in between the
 * blocks; no explicit inverse. alpha == 0 sets B to zero without reading A
 * or B. Replaces strsm (src/strsm/strsm.mjs:148-583). */
int wgb_strsm(wgb_ctx *ctx, int side, int uplo, int transA, int diag,
              int64_t m, int64_t n, float alpha, const float *A, int64_t lda,
              float *B, int64_t ldb);

/* ---- level 2 -------------------------------------------------------------- */

/* y <- alpha*op(A)*x + beta*y, A m-by-n column-major: op(A) = A (trans ==
 * WGB_NO_TRANS: x of length n, y of length m) or A^T (x of length m, y of
 * length n). Reference BLAS rules: m == 0, n == 0, or alpha == 0 with
 * beta == 1 leave y untouched; alpha == 0 reads neither A nor x; beta == 0
 * never reads y; the WGB_NO_TRANS form skips a column whose x entry is zero
 * (its Inf / NaN entries never reach y), the transposed form takes every
 * term. Replaces sgemv (src/sgemv/sgemv.mjs:19-254, src/shaders/sgemv_n.wgsl,
 * sgemv_t.wgsl, reduce_partials.wgsl). */
int wgb_sgemv(wgb_ctx *ctx, int trans, int64_t m, int64_t n, float alpha,
              const float *A, int64_t lda, const float *x, int64_t incx,
              float beta, float *y, int64_t incy);

/* A <- alpha*x*y^T + A, A m-by-n column-major, x of length m, y of length
 * n. Reference BLAS rules: m == 0, n == 0 or alpha == 0 leave A untouched
 * and read neither x nor y; a column whose y entry is zero is skipped (its
 * A entries are neither computed nor written, so Inf / NaN in x never meets
 * that zero); otherwise A(i,j) = fma(x(i), alpha*y(j), A(i,j)). Replaces
 * sger (src/sger/sger.mjs:17-176, src/shaders/sger.wgsl; its row-major
 * frame skips rows where x is zero, this column-major y after the layout
 * swap of sger.mjs:56-64). */
int wgb_sger(wgb_ctx *ctx, int64_t m, int64_t n, float alpha, const float *x,
             int64_t incx, const float *y, int64_t incy, float *A, int64_t lda);

/* Native-FP64 dger: wgb_sger in fp64. Replaces dger (src/dger/dger.mjs:21-238,
 * src/shaders/dger.wgsl in double-double). */
int wgb_dger(wgb_ctx *ctx, int64_t m, int64_t n, double alpha, const double *x,
             int64_t incx, const double *y, int64_t incy, double *A, int64_t lda);

/* The uplo triangle (WGB_LOWER: i >= j, WGB_UPPER: i <= j) of the n-by-n
 * column-major A <- alpha*x*x^T + A; the other triangle is never written
 * (its values never reach the result). Reference BLAS rules: n == 0 or alpha == 0 leave A untouched and
 * read no vector; a column whose x entry is zero is skipped (Inf / NaN in x
 * never meets it); otherwise A(i,j) = fma(x(i), alpha*x(j), A(i,j)).
 * Replaces ssyr (src/ssyr/ssyr.mjs:17-143, src/shaders/ssyr.wgsl; its
 * row-major frame skips rows, this column after the uplo flip of
 * ssyr.mjs:68-71). */
int wgb_ssyr(wgb_ctx *ctx, int uplo, int64_t n, float alpha, const float *x,
             int64_t incx, float *A, int64_t lda);

/* Native-FP64 dsyr: wgb_ssyr in fp64. Replaces dsyr
 * (src/dsyr/dsyr.mjs:21-196, double-double in dsyr.wgsl). */
int wgb_dsyr(wgb_ctx *ctx, int uplo, int64_t n, double alpha, const double *x,
             int64_t incx, double *A, int64_t lda);

/* The uplo triangle of A <- alpha*x*y^T + alpha*y*x^T + A (n-by-n,
 * column-major); column j is skipped when x(j) and y(j) are both zero,
 * otherwise A(i,j) = fma(y(i), alpha*x(j), fma(x(i), alpha*y(j), A(i,j))).
 * n == 0 or alpha == 0 leave A untouched. Replaces ssyr2
 * (src/ssyr2/ssyr2.mjs:17-184, src/shaders/ssyr2.wgsl). */
int wgb_ssyr2(wgb_ctx *ctx, int uplo, int64_t n, float alpha, const float *x,
              int64_t incx, const float *y, int64_t incy, float *A,
              int64_t lda);

/* Native-FP64 dsyr2: wgb_ssyr2 in fp64. Replaces dsyr2
 * (src/dsyr2/dsyr2.mjs:21-260, double-double in dsyr2.wgsl). */
int wgb_dsyr2(wgb_ctx *ctx, int uplo, int64_t n, double alpha,
              const double *x, int64_t incx, const double *y, int64_t incy,
              double *A, int64_t lda);

/* y <- alpha*S*x + beta*y, S the n-by-n symmetric matrix whose uplo
 * triangle (WGB_LOWER / WGB_UPPER) the column-major A holds; the other
 * triangle is never read. Reference BLAS rules: n == 0, or alpha == 0 with
 * beta == 1, leave y untouched; alpha == 0 reads neither A nor x; beta == 0
 * never reads y; every term is taken. The triangle is read once; partial
 * sums are folded in a fixed order (deterministic). Replaces ssymv
 * (src/ssymv/ssymv.mjs:17-216, src/shaders/ssymv.wgsl, reduce_partials.wgsl). */
int wgb_ssymv(wgb_ctx *ctx, int uplo, int64_t n, float alpha, const float *A,
              int64_t lda, const float *x, int64_t incx, float beta, float *y,
              int64_t incy);

/* Native-FP64 dsymv: wgb_ssymv in fp64, alpha == 0 with beta == 1 returning
 * without a kernel (src/dsymv/dsymv.mjs:116). Replaces dsymv
 * (src/dsymv/dsymv.mjs:25-336, double-double in dsymv.wgsl). */
int wgb_dsymv(wgb_ctx *ctx, int uplo, int64_t n, double alpha, const double *A,
              int64_t lda, const double *x, int64_t incx, double beta,
              double *y, int64_t incy);

/* strmv: y <- op(T) x out of place, T the n x n uplo triangle of the
 * column-major A (lda >= max(1, n)), op(T) = T (WGB_NO_TRANS) or T^T
 * (WGB_TRANS), diag WGB_UNIT taking the diagonal as 1 (never read); incx,
 * incy > 0; y is written, never read, and must not overlap A or x. The
 * WGB_NO_TRANS form skips a column whose x entry is zero (reference BLAS's
 * column form), the transposed one takes every term. One pass over the
 * triangle (row or column sums of 1024 x 128 blocks), then a fixed-order
 * fold (deterministic). Replaces strmv (src/strmv/strmv.mjs:20-259,
 * src/shaders/strmv.wgsl, strmv_t.wgsl, reduce_partials.wgsl). */
int wgb_strmv(wgb_ctx *ctx, int uplo, int trans, int diag, int64_t n,
              const float *A, int64_t lda, const float *x, int64_t incx,
              float *y, int64_t incy);

/* Native-FP64 dtrmv: wgb_strmv in fp64. Replaces dtrmv
 * (src/dtrmv/dtrmv.mjs:24-355, double-double in dtrmv.wgsl, dtrmv_t.wgsl). */
int wgb_dtrmv(wgb_ctx *ctx, int uplo, int trans, int diag, int64_t n,
              const double *A, int64_t lda, const double *x, int64_t incx,
              double *y, int64_t incy);

/* Native-FP64 dgemv: wgb_sgemv's operation and rules in fp64 (alpha == 0
 * with beta == 1 returns without a kernel, src/dgemv/dgemv.mjs:126).
 * Replaces dgemv (src/dgemv/dgemv.mjs:23-341, src/shaders/dgemv_n.wgsl,
 * dgemv_t.wgsl, reduce_partials_f64.wgsl in double-double). */
int wgb_dgemv(wgb_ctx *ctx, int trans, int64_t m, int64_t n, double alpha,
              const double *A, int64_t lda, const double *x, int64_t incx,
              double beta, double *y, int64_t incy);

/* ---- level 1 reductions --------------------------------------------------- */
/* n <= 0 returns 0 (index -1) without touching the device. incx, incy must be
 * positive. The host-result forms block until the value is on the host; the
 * `_dev` forms write the result to device memory and return without
 * synchronising. Both run a fixed two-pass reduction whose summation order
 * depends only on n, so results are reproducible run to run. */

/* sum x[i*incx]*y[i*incy] in float32. Replaces sdot (src/sdot/sdot.mjs:18-117,
 * src/shaders/sdot.wgsl, src/shaders/reduction/sum.wgsl). */
int wgb_sdot(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx,
             const float *y, int64_t incy, float *result);
int wgb_sdot_dev(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx,
                 const float *y, int64_t incy, float *d_result);

/* sum |x[i*incx]|. Replaces sasum (src/sasum/sasum.mjs, src/shaders/sasum.wgsl). */
int wgb_sasum(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx,
              float *result);
int wgb_sasum_dev(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx,
                  float *d_result);

/* Overflow-safe Euclidean norm: Blue's three accumulators with wgblas's
 * thresholds and LAPACK 3.10 combine. Replaces snrm2 (src/snrm2/snrm2.mjs,
 * src/shaders/snrm2.wgsl, src/shaders/reduction/scaledSum.wgsl). */
int wgb_snrm2(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx,
              float *result);
int wgb_snrm2_dev(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx,
                  float *d_result);

/* 0-based logical index of the first max |x[i*incx]|; NaN never wins, an
 * all-NaN vector gives 0, n <= 0 gives -1. Replaces isamax
 * (src/isamax/isamax.mjs, src/shaders/isamax.wgsl,
 * src/shaders/reduction/argmax.wgsl). */
int wgb_isamax(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx,
               int64_t *result);
int wgb_isamax_dev(wgb_ctx *ctx, int64_t n, const float *x, int64_t incx,
                   int64_t *d_result);

/* The fp64 reductions, accumulated in native float64 with the same rules as
 * their fp32 counterparts (wgblas computes them in double-double:
 * src/shaders/{ddot,dasum,dnrm2,idamax}.wgsl, src/shaders/reduction/(name)F64.wgsl).
 * ddot replaces src/ddot/ddot.mjs:19-174; dasum src/dasum/dasum.mjs:18-138;
 * dnrm2 src/dnrm2/dnrm2.mjs:22-149 (Blue's algorithm with LAPACK 3.10's
 * dnrm2 thresholds for IEEE double; NaN gives NaN, Inf gives Inf); idamax
 * src/idamax/idamax.mjs:18-152 (isamax's NaN and tie rules, n <= 0 -> -1). */
int wgb_ddot(wgb_ctx *ctx, int64_t n, const double *x, int64_t incx,
             const double *y, int64_t incy, double *result);
int wgb_ddot_dev(wgb_ctx *ctx, int64_t n, const double *x, int64_t incx,
                 const double *y, int64_t incy, double *d_result);
int wgb_dasum(wgb_ctx *ctx, int64_t n, const double *x, int64_t incx,
              double *result);
int wgb_dasum_dev(wgb_ctx *ctx, int64_t n, const double *x, int64_t incx,
                  double *d_result);
int wgb_dnrm2(wgb_ctx *ctx, int64_t n, const double *x, int64_t incx,
              double *result);
int wgb_dnrm2_dev(wgb_ctx *ctx, int64_t n, const double *x, int64_t incx,
                  double *d_result);
int wgb_idamax(wgb_ctx *ctx, int64_t n, const double *x, int64_t incx,
               int64_t *result);
int wgb_idamax_dev(wgb_ctx *ctx, int64_t n, const double *x, int64_t incx,
                   int64_t *d_result);

#ifdef __cplusplus
}
#endif

#endif /* WGBLAS_HIP_H */
