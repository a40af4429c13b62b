// Node-API addon: the JavaScript side of wgblas binds the C ABI of
// libwgblas_hip (include/wgblas_hip.h) through these functions. Each one
// converts its arguments, calls one wgb_* entry point and turns a failing
// status into a thrown Error carrying wgb_last_error(). Device pointers
// travel to JavaScript as napi_external values; the JavaScript classes
// (GpuVector, GpuMatrix, the device handle) own them and free them.
#include <node_api.h>

#include <cstdint>
#include <cstring>
#include <set>
#include <string>

#include "wgblas_hip.h"

namespace {

#define NAPI_OK(call)                                          \
  do {                                                         \
    if ((call) != napi_ok) {                                   \
      napi_throw_error(env, nullptr, "wgblas_hip addon: " #call); \
      return nullptr;                                          \
    }                                                          \
  } while (0)

napi_value throw_status(napi_env env, int status, const char *what) {
  std::string msg = std::string(what) + " failed (" + wgb_status_string(status) + "): " + wgb_last_error();
  napi_throw_error(env, nullptr, msg.c_str());
  return nullptr;
}

#define WGB_OK_OR_THROW(call, what)               \
  do {                                            \
    int _st = (call);                             \
    if (_st != WGB_OK) return throw_status(env, _st, what); \
  } while (0)

struct Args {
  napi_value v[16];
  size_t n = 16;
};

bool get_args(napi_env env, napi_callback_info info, Args &a, size_t want) {
  a.n = 16;
  if (napi_get_cb_info(env, info, &a.n, a.v, nullptr, nullptr) != napi_ok) return false;
  if (a.n < want) {
    napi_throw_type_error(env, nullptr, "wgblas_hip addon: too few arguments");
    return false;
  }
  return true;
}

bool get_ptr(napi_env env, napi_value v, void **out) {
  napi_valuetype t;
  if (napi_typeof(env, v, &t) != napi_ok) return false;
  if (t == napi_null || t == napi_undefined) {
    *out = nullptr;
    return true;
  }
  if (t != napi_external) {
    napi_throw_type_error(env, nullptr, "wgblas_hip addon: expected a device handle");
    return false;
  }
  return napi_get_value_external(env, v, out) == napi_ok;
}

bool get_i64(napi_env env, napi_value v, int64_t *out) {
  if (napi_get_value_int64(env, v, out) != napi_ok) {
    napi_throw_type_error(env, nullptr, "wgblas_hip addon: expected an integer");
    return false;
  }
  return true;
}

bool get_f64(napi_env env, napi_value v, double *out) {
  if (napi_get_value_double(env, v, out) != napi_ok) {
    napi_throw_type_error(env, nullptr, "wgblas_hip addon: expected a number");
    return false;
  }
  return true;
}

bool get_i32(napi_env env, napi_value v, int *out) {
  int32_t x;
  if (napi_get_value_int32(env, v, &x) != napi_ok) {
    napi_throw_type_error(env, nullptr, "wgblas_hip addon: expected an int32");
    return false;
  }
  *out = x;
  return true;
}

// (data pointer, byte length) of a TypedArray.
bool get_typed(napi_env env, napi_value v, void **data, size_t *bytes) {
  bool is_ta = false;
  if (napi_is_typedarray(env, v, &is_ta) != napi_ok || !is_ta) {
    napi_throw_type_error(env, nullptr, "wgblas_hip addon: expected a TypedArray");
    return false;
  }
  napi_typedarray_type type;
  size_t length, offset;
  napi_value ab;
  void *base;
  if (napi_get_typedarray_info(env, v, &type, &length, &base, &ab, &offset) != napi_ok) return false;
  size_t elem = 1;
  switch (type) {
    case napi_float32_array: case napi_int32_array: case napi_uint32_array: elem = 4; break;
    case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: elem = 8; break;
    case napi_int16_array: case napi_uint16_array: elem = 2; break;
    default: elem = 1; break;
  }
  *data = base;  // already points at the view's first element
  *bytes = length * elem;
  return true;
}

napi_value make_external(napi_env env, void *p) {
  napi_value out;
  if (napi_create_external(env, p, nullptr, nullptr, &out) != napi_ok) return nullptr;
  return out;
}

napi_value num(napi_env env, double d) {
  napi_value out;
  napi_create_double(env, d, &out);
  return out;
}

wgb_ctx *ctx_of(napi_env env, napi_value v) {
  void *p = nullptr;
  if (!get_ptr(env, v, &p)) return nullptr;
  if (!p) napi_throw_error(env, nullptr, "wgblas_hip addon: device handle was released (cleanup() called?)");
  return (wgb_ctx *)p;
}

// ---- device ----------------------------------------------------------------

// Contexts created through this addon and not yet destroyed. The JavaScript
// layer releases them in cleanup(); any still open when the Node environment
// is torn down (a program that never called cleanup()) are destroyed by the
// environment's cleanup hook, which Node runs before the process's exit
// handlers, so no stream, event or buffer of the library is left for the
// HIP runtime's own exit-time teardown.
std::set<wgb_ctx *> &live_contexts() {
  static std::set<wgb_ctx *> live;
  return live;
}

void destroy_live_contexts(void *) {
  std::set<wgb_ctx *> &live = live_contexts();
  for (wgb_ctx *ctx : live) (void)wgb_destroy(ctx);
  live.clear();
}

napi_value DeviceCount(napi_env env, napi_callback_info) {
  int c = 0;
  WGB_OK_OR_THROW(wgb_device_count(&c), "wgb_device_count");
  return num(env, c);
}

napi_value Init(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  int dev;
  if (!get_i32(env, a.v[0], &dev)) return nullptr;
  wgb_ctx *ctx = nullptr;
  WGB_OK_OR_THROW(wgb_init(dev, &ctx), "wgb_init");
  live_contexts().insert(ctx);
  return make_external(env, ctx);
}

napi_value Destroy(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  void *p;
  if (!get_ptr(env, a.v[0], &p)) return nullptr;
  // Only contexts this addon created and has not destroyed yet: a second
  // destroy of the same handle is a no-op instead of a double free.
  if (live_contexts().erase((wgb_ctx *)p) == 0) return nullptr;
  WGB_OK_OR_THROW(wgb_destroy((wgb_ctx *)p), "wgb_destroy");
  return nullptr;
}

napi_value DeviceName(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[0]);
  if (!ctx) return nullptr;
  char name[256], arch[64];
  WGB_OK_OR_THROW(wgb_device_name(ctx, name, sizeof name, arch, sizeof arch), "wgb_device_name");
  napi_value obj, s1, s2;
  NAPI_OK(napi_create_object(env, &obj));
  NAPI_OK(napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &s1));
  NAPI_OK(napi_create_string_utf8(env, arch, NAPI_AUTO_LENGTH, &s2));
  NAPI_OK(napi_set_named_property(env, obj, "name", s1));
  NAPI_OK(napi_set_named_property(env, obj, "arch", s2));
  return obj;
}

napi_value SetTiming(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[0]);
  if (!ctx) return nullptr;
  bool on = false;
  NAPI_OK(napi_get_value_bool(env, a.v[1], &on));
  WGB_OK_OR_THROW(wgb_set_timing(ctx, on ? 1 : 0), "wgb_set_timing");
  return nullptr;
}

napi_value LastTimeMs(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[0]);
  if (!ctx) return nullptr;
  float ms = 0;
  WGB_OK_OR_THROW(wgb_last_time_ms(ctx, &ms), "wgb_last_time_ms");
  return num(env, ms);
}

napi_value Synchronize(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[0]);
  if (!ctx) return nullptr;
  WGB_OK_OR_THROW(wgb_synchronize(ctx), "wgb_synchronize");
  return nullptr;
}

// ---- memory ------------------------------------------------------------------

napi_value Malloc(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[0]);
  if (!ctx) return nullptr;
  int64_t bytes;
  if (!get_i64(env, a.v[1], &bytes)) return nullptr;
  if (bytes < 0) {
    napi_throw_range_error(env, nullptr, "wgblas_hip addon: negative allocation size");
    return nullptr;
  }
  void *p = nullptr;
  WGB_OK_OR_THROW(wgb_malloc(ctx, (size_t)bytes, &p), "wgb_malloc");
  return make_external(env, p);
}

napi_value Free(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[0]);
  if (!ctx) return nullptr;
  void *p;
  if (!get_ptr(env, a.v[1], &p)) return nullptr;
  WGB_OK_OR_THROW(wgb_free(ctx, p), "wgb_free");
  return nullptr;
}

// upload(ctx, dptr, typedArray[, byteOffset]): whole TypedArray -> device.
napi_value Upload(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[0]);
  if (!ctx) return nullptr;
  void *dptr, *host;
  size_t bytes;
  if (!get_ptr(env, a.v[1], &dptr) || !get_typed(env, a.v[2], &host, &bytes)) return nullptr;
  int64_t off = 0;
  if (a.n > 3 && !get_i64(env, a.v[3], &off)) return nullptr;
  WGB_OK_OR_THROW(wgb_memcpy_h2d(ctx, (char *)dptr + off, host, bytes), "wgb_memcpy_h2d");
  return nullptr;
}

// download(ctx, dptr, typedArray[, byteOffset]): device -> whole TypedArray.
napi_value Download(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[0]);
  if (!ctx) return nullptr;
  void *dptr, *host;
  size_t bytes;
  if (!get_ptr(env, a.v[1], &dptr) || !get_typed(env, a.v[2], &host, &bytes)) return nullptr;
  int64_t off = 0;
  if (a.n > 3 && !get_i64(env, a.v[3], &off)) return nullptr;
  WGB_OK_OR_THROW(wgb_memcpy_d2h(ctx, host, (const char *)dptr + off, bytes), "wgb_memcpy_d2h");
  return nullptr;
}

// ---- level 3 ---------------------------------------------------------------

// gemm(kind, ctx, uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc)
// kind: 0 sgemm, 1 sgemmtr, 2 dgemm, 3 dgemmtr.
napi_value Gemm(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 16)) return nullptr;
  int kind, uplo, ta, tb;
  int64_t m, n, k, lda, ldb, ldc;
  double alpha, beta;
  void *A, *B, *C;
  if (!get_i32(env, a.v[0], &kind)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[1]);
  if (!ctx) return nullptr;
  if (!get_i32(env, a.v[2], &uplo) || !get_i32(env, a.v[3], &ta) || !get_i32(env, a.v[4], &tb) ||
      !get_i64(env, a.v[5], &m) || !get_i64(env, a.v[6], &n) || !get_i64(env, a.v[7], &k) ||
      !get_f64(env, a.v[8], &alpha) || !get_ptr(env, a.v[9], &A) || !get_i64(env, a.v[10], &lda) ||
      !get_ptr(env, a.v[11], &B) || !get_i64(env, a.v[12], &ldb) || !get_f64(env, a.v[13], &beta) ||
      !get_ptr(env, a.v[14], &C) || !get_i64(env, a.v[15], &ldc))
    return nullptr;
  if (kind == 0) {
    WGB_OK_OR_THROW(wgb_sgemm(ctx, ta, tb, m, n, k, (float)alpha, (const float *)A, lda,
                              (const float *)B, ldb, (float)beta, (float *)C, ldc), "wgb_sgemm");
  } else if (kind == 1) {
    WGB_OK_OR_THROW(wgb_sgemmtr(ctx, uplo, ta, tb, m, n, k, (float)alpha, (const float *)A, lda,
                                (const float *)B, ldb, (float)beta, (float *)C, ldc), "wgb_sgemmtr");
  } else if (kind == 2) {
    WGB_OK_OR_THROW(wgb_dgemm(ctx, ta, tb, m, n, k, alpha, (const double *)A, lda,
                              (const double *)B, ldb, beta, (double *)C, ldc), "wgb_dgemm");
  } else {
    WGB_OK_OR_THROW(wgb_dgemmtr(ctx, uplo, ta, tb, m, n, k, alpha, (const double *)A, lda,
                                (const double *)B, ldb, beta, (double *)C, ldc), "wgb_dgemmtr");
  }
  return nullptr;
}

// syrk(ctx, uplo, trans, n, k, alpha, A, lda, beta, C, ldc[, f64]): ssyrk, or
// dsyrk when the optional twelfth argument is true.
napi_value Ssyrk(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 11)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[0]);
  if (!ctx) return nullptr;
  int uplo, trans;
  int64_t n, k, lda, ldc;
  double alpha, beta;
  void *A, *C;
  if (!get_i32(env, a.v[1], &uplo) || !get_i32(env, a.v[2], &trans) || !get_i64(env, a.v[3], &n) ||
      !get_i64(env, a.v[4], &k) || !get_f64(env, a.v[5], &alpha) || !get_ptr(env, a.v[6], &A) ||
      !get_i64(env, a.v[7], &lda) || !get_f64(env, a.v[8], &beta) || !get_ptr(env, a.v[9], &C) ||
      !get_i64(env, a.v[10], &ldc))
    return nullptr;
  bool f64 = false;
  if (a.n > 11 && napi_get_value_bool(env, a.v[11], &f64) != napi_ok) f64 = false;
  if (f64) {
    WGB_OK_OR_THROW(wgb_dsyrk(ctx, uplo, trans, n, k, alpha, (const double *)A, lda, beta,
                              (double *)C, ldc), "wgb_dsyrk");
  } else {
    WGB_OK_OR_THROW(wgb_ssyrk(ctx, uplo, trans, n, k, (float)alpha, (const float *)A, lda,
                              (float)beta, (float *)C, ldc), "wgb_ssyrk");
  }
  return nullptr;
}

// ssyr2k(ctx, uplo, transA, transB, n, k, alpha, A, lda, B, ldb, beta, C, ldc)
napi_value Ssyr2k(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 14)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[0]);
  if (!ctx) return nullptr;
  int uplo, ta, tb;
  int64_t n, k, lda, ldb, ldc;
  double alpha, beta;
  void *A, *B, *C;
  if (!get_i32(env, a.v[1], &uplo) || !get_i32(env, a.v[2], &ta) || !get_i32(env, a.v[3], &tb) ||
      !get_i64(env, a.v[4], &n) || !get_i64(env, a.v[5], &k) || !get_f64(env, a.v[6], &alpha) ||
      !get_ptr(env, a.v[7], &A) || !get_i64(env, a.v[8], &lda) || !get_ptr(env, a.v[9], &B) ||
      !get_i64(env, a.v[10], &ldb) || !get_f64(env, a.v[11], &beta) || !get_ptr(env, a.v[12], &C) ||
      !get_i64(env, a.v[13], &ldc))
    return nullptr;
  bool f64 = false;  // optional 15th argument: dsyr2k
  if (a.n > 14 && napi_get_value_bool(env, a.v[14], &f64) != napi_ok) f64 = false;
  if (f64) {
    WGB_OK_OR_THROW(wgb_dsyr2k(ctx, uplo, ta, tb, n, k, alpha, (const double *)A, lda,
                               (const double *)B, ldb, beta, (double *)C, ldc), "wgb_dsyr2k");
  } else {
    WGB_OK_OR_THROW(wgb_ssyr2k(ctx, uplo, ta, tb, n, k, (float)alpha, (const float *)A, lda,
                               (const float *)B, ldb, (float)beta, (float *)C, ldc), "wgb_ssyr2k");
  }
  return nullptr;
}

// ssymm(ctx, side, uplo, transB, m, n, alpha, A, lda, B, ldb, beta, C, ldc)
napi_value Ssymm(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 14)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[0]);
  if (!ctx) return nullptr;
  int side, uplo, tb;
  int64_t m, n, lda, ldb, ldc;
  double alpha, beta;
  void *A, *B, *C;
  if (!get_i32(env, a.v[1], &side) || !get_i32(env, a.v[2], &uplo) || !get_i32(env, a.v[3], &tb) ||
      !get_i64(env, a.v[4], &m) || !get_i64(env, a.v[5], &n) || !get_f64(env, a.v[6], &alpha) ||
      !get_ptr(env, a.v[7], &A) || !get_i64(env, a.v[8], &lda) || !get_ptr(env, a.v[9], &B) ||
      !get_i64(env, a.v[10], &ldb) || !get_f64(env, a.v[11], &beta) || !get_ptr(env, a.v[12], &C) ||
      !get_i64(env, a.v[13], &ldc))
    return nullptr;
  bool f64 = false;  // optional 15th argument: dsymm
  if (a.n > 14 && napi_get_value_bool(env, a.v[14], &f64) != napi_ok) f64 = false;
  if (f64) {
    WGB_OK_OR_THROW(wgb_dsymm(ctx, side, uplo, tb, m, n, alpha, (const double *)A, lda,
                              (const double *)B, ldb, beta, (double *)C, ldc), "wgb_dsymm");
  } else {
    WGB_OK_OR_THROW(wgb_ssymm(ctx, side, uplo, tb, m, n, (float)alpha, (const float *)A, lda,
                              (const float *)B, ldb, (float)beta, (float *)C, ldc), "wgb_ssymm");
  }
  return nullptr;
}

// tri(kind, ctx, side, uplo, transA, diag, m, n, alpha, A, lda, B, ldb);
// kind: 0 strmm, 1 strsm, 2 dtrmm.
napi_value Tri(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 13)) return nullptr;
  int kind, side, uplo, trans, diag;
  if (!get_i32(env, a.v[0], &kind)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[1]);
  if (!ctx) return nullptr;
  int64_t m, n, lda, ldb;
  double alpha;
  void *A, *B;
  if (!get_i32(env, a.v[2], &side) || !get_i32(env, a.v[3], &uplo) || !get_i32(env, a.v[4], &trans) ||
      !get_i32(env, a.v[5], &diag) || !get_i64(env, a.v[6], &m) || !get_i64(env, a.v[7], &n) ||
      !get_f64(env, a.v[8], &alpha) || !get_ptr(env, a.v[9], &A) || !get_i64(env, a.v[10], &lda) ||
      !get_ptr(env, a.v[11], &B) || !get_i64(env, a.v[12], &ldb))
    return nullptr;
  if (kind == 0) {
    WGB_OK_OR_THROW(wgb_strmm(ctx, side, uplo, trans, diag, m, n, (float)alpha, (const float *)A,
                              lda, (float *)B, ldb), "wgb_strmm");
  } else if (kind == 2) {
    WGB_OK_OR_THROW(wgb_dtrmm(ctx, side, uplo, trans, diag, m, n, alpha, (const double *)A, lda,
                              (double *)B, ldb), "wgb_dtrmm");
  } else {
    WGB_OK_OR_THROW(wgb_strsm(ctx, side, uplo, trans, diag, m, n, (float)alpha, (const float *)A,
                              lda, (float *)B, ldb), "wgb_strsm");
  }
  return nullptr;
}

// ---- level 2 ---------------------------------------------------------------

// sgemv(ctx, trans, m, n, alpha, A, lda, x, incx, beta, y, incy[, f64]):
// sgemv, or dgemv when f64 is true
napi_value Sgemv(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 12)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[0]);
  if (!ctx) return nullptr;
  int trans;
  int64_t m, n, lda, incx, incy;
  double alpha, beta;
  void *A, *x, *y;
  if (!get_i32(env, a.v[1], &trans) || !get_i64(env, a.v[2], &m) || !get_i64(env, a.v[3], &n) ||
      !get_f64(env, a.v[4], &alpha) || !get_ptr(env, a.v[5], &A) || !get_i64(env, a.v[6], &lda) ||
      !get_ptr(env, a.v[7], &x) || !get_i64(env, a.v[8], &incx) || !get_f64(env, a.v[9], &beta) ||
      !get_ptr(env, a.v[10], &y) || !get_i64(env, a.v[11], &incy))
    return nullptr;
  bool f64 = false;
  if (a.n > 12 && napi_get_value_bool(env, a.v[12], &f64) != napi_ok) f64 = false;
  if (f64) {
    WGB_OK_OR_THROW(wgb_dgemv(ctx, trans, m, n, alpha, (const double *)A, lda, (const double *)x,
                              incx, beta, (double *)y, incy), "wgb_dgemv");
  } else {
    WGB_OK_OR_THROW(wgb_sgemv(ctx, trans, m, n, (float)alpha, (const float *)A, lda,
                              (const float *)x, incx, (float)beta, (float *)y, incy), "wgb_sgemv");
  }
  return nullptr;
}

// ger(ctx, m, n, alpha, x, incx, y, incy, A, lda, f64): sger, or dger when
// f64 is true
napi_value Ger(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 11)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[0]);
  if (!ctx) return nullptr;
  int64_t m, n, incx, incy, lda;
  double alpha;
  void *x, *y, *A;
  bool f64 = false;
  if (!get_i64(env, a.v[1], &m) || !get_i64(env, a.v[2], &n) || !get_f64(env, a.v[3], &alpha) ||
      !get_ptr(env, a.v[4], &x) || !get_i64(env, a.v[5], &incx) || !get_ptr(env, a.v[6], &y) ||
      !get_i64(env, a.v[7], &incy) || !get_ptr(env, a.v[8], &A) || !get_i64(env, a.v[9], &lda) ||
      napi_get_value_bool(env, a.v[10], &f64) != napi_ok)
    return nullptr;
  if (f64) {
    WGB_OK_OR_THROW(wgb_dger(ctx, m, n, alpha, (const double *)x, incx, (const double *)y, incy,
                             (double *)A, lda), "wgb_dger");
  } else {
    WGB_OK_OR_THROW(wgb_sger(ctx, m, n, (float)alpha, (const float *)x, incx, (const float *)y,
                             incy, (float *)A, lda), "wgb_sger");
  }
  return nullptr;
}

// syr(ctx, uplo, n, alpha, x, incx, y, incy, A, lda, f64): ssyr2 / dsyr2, or
// ssyr / dsyr when y is null
napi_value Syr(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 11)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[0]);
  if (!ctx) return nullptr;
  int uplo;
  int64_t n, incx, incy, lda;
  double alpha;
  void *x, *A, *y;
  bool f64 = false;
  if (!get_i32(env, a.v[1], &uplo) || !get_i64(env, a.v[2], &n) || !get_f64(env, a.v[3], &alpha) ||
      !get_ptr(env, a.v[4], &x) || !get_i64(env, a.v[5], &incx) || !get_ptr(env, a.v[6], &y) ||
      !get_i64(env, a.v[7], &incy) || !get_ptr(env, a.v[8], &A) || !get_i64(env, a.v[9], &lda) ||
      napi_get_value_bool(env, a.v[10], &f64) != napi_ok)
    return nullptr;
  if (y == nullptr) {
    if (f64)
      WGB_OK_OR_THROW(wgb_dsyr(ctx, uplo, n, alpha, (const double *)x, incx, (double *)A, lda),
                      "wgb_dsyr");
    else
      WGB_OK_OR_THROW(wgb_ssyr(ctx, uplo, n, (float)alpha, (const float *)x, incx, (float *)A, lda),
                      "wgb_ssyr");
  } else if (f64) {
    WGB_OK_OR_THROW(wgb_dsyr2(ctx, uplo, n, alpha, (const double *)x, incx, (const double *)y, incy,
                              (double *)A, lda), "wgb_dsyr2");
  } else {
    WGB_OK_OR_THROW(wgb_ssyr2(ctx, uplo, n, (float)alpha, (const float *)x, incx, (const float *)y,
                              incy, (float *)A, lda), "wgb_ssyr2");
  }
  return nullptr;
}

// symv(ctx, uplo, n, alpha, A, lda, x, incx, beta, y, incy, f64): ssymv, or
// dsymv when f64 is true
napi_value Symv(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 12)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[0]);
  if (!ctx) return nullptr;
  int uplo;
  int64_t n, lda, incx, incy;
  double alpha, beta;
  void *A, *x, *y;
  bool f64 = false;
  if (!get_i32(env, a.v[1], &uplo) || !get_i64(env, a.v[2], &n) || !get_f64(env, a.v[3], &alpha) ||
      !get_ptr(env, a.v[4], &A) || !get_i64(env, a.v[5], &lda) || !get_ptr(env, a.v[6], &x) ||
      !get_i64(env, a.v[7], &incx) || !get_f64(env, a.v[8], &beta) || !get_ptr(env, a.v[9], &y) ||
      !get_i64(env, a.v[10], &incy) || napi_get_value_bool(env, a.v[11], &f64) != napi_ok)
    return nullptr;
  if (f64) {
    WGB_OK_OR_THROW(wgb_dsymv(ctx, uplo, n, alpha, (const double *)A, lda, (const double *)x, incx,
                              beta, (double *)y, incy), "wgb_dsymv");
  } else {
    WGB_OK_OR_THROW(wgb_ssymv(ctx, uplo, n, (float)alpha, (const float *)A, lda, (const float *)x,
                              incx, (float)beta, (float *)y, incy), "wgb_ssymv");
  }
  return nullptr;
}

// trmv(ctx, uplo, trans, diag, n, A, lda, x, incx, y, incy, f64): strmv, or
// dtrmv when f64 is true
napi_value Trmv(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 12)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[0]);
  if (!ctx) return nullptr;
  int uplo, trans, diag;
  int64_t n, lda, incx, incy;
  void *A, *x, *y;
  bool f64 = false;
  if (!get_i32(env, a.v[1], &uplo) || !get_i32(env, a.v[2], &trans) || !get_i32(env, a.v[3], &diag) ||
      !get_i64(env, a.v[4], &n) || !get_ptr(env, a.v[5], &A) || !get_i64(env, a.v[6], &lda) ||
      !get_ptr(env, a.v[7], &x) || !get_i64(env, a.v[8], &incx) || !get_ptr(env, a.v[9], &y) ||
      !get_i64(env, a.v[10], &incy) || napi_get_value_bool(env, a.v[11], &f64) != napi_ok)
    return nullptr;
  if (f64) {
    WGB_OK_OR_THROW(wgb_dtrmv(ctx, uplo, trans, diag, n, (const double *)A, lda, (const double *)x, incx,
                              (double *)y, incy), "wgb_dtrmv");
  } else {
    WGB_OK_OR_THROW(wgb_strmv(ctx, uplo, trans, diag, n, (const float *)A, lda, (const float *)x, incx,
                              (float *)y, incy), "wgb_strmv");
  }
  return nullptr;
}

// ---- level 1 ---------------------------------------------------------------

// reduce(kind, ctx, n, x, incx[, y, incy]) -> number; kind: 0 sdot, 1 sasum,
// 2 snrm2, 3 isamax, 4 ddot, 5 dasum, 6 dnrm2, 7 idamax.
napi_value Reduce(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 5)) return nullptr;
  int kind;
  if (!get_i32(env, a.v[0], &kind)) return nullptr;
  wgb_ctx *ctx = ctx_of(env, a.v[1]);
  if (!ctx) return nullptr;
  int64_t n, incx, incy = 1;
  void *x, *y = nullptr;
  if (!get_i64(env, a.v[2], &n) || !get_ptr(env, a.v[3], &x) || !get_i64(env, a.v[4], &incx))
    return nullptr;
  if (kind == 0 || kind == 4) {
    if (a.n < 7) {
      napi_throw_type_error(env, nullptr, "wgblas_hip addon: sdot / ddot need y and incy");
      return nullptr;
    }
    if (!get_ptr(env, a.v[5], &y) || !get_i64(env, a.v[6], &incy)) return nullptr;
  }
  float r = 0;
  double d = 0;
  int64_t idx = -1;
  const double *xd = (const double *)x;
  switch (kind) {
    case 0: WGB_OK_OR_THROW(wgb_sdot(ctx, n, (const float *)x, incx, (const float *)y, incy, &r), "wgb_sdot"); break;
    case 1: WGB_OK_OR_THROW(wgb_sasum(ctx, n, (const float *)x, incx, &r), "wgb_sasum"); break;
    case 2: WGB_OK_OR_THROW(wgb_snrm2(ctx, n, (const float *)x, incx, &r), "wgb_snrm2"); break;
    case 3: WGB_OK_OR_THROW(wgb_isamax(ctx, n, (const float *)x, incx, &idx), "wgb_isamax"); return num(env, (double)idx);
    case 4: WGB_OK_OR_THROW(wgb_ddot(ctx, n, xd, incx, (const double *)y, incy, &d), "wgb_ddot"); return num(env, d);
    case 5: WGB_OK_OR_THROW(wgb_dasum(ctx, n, xd, incx, &d), "wgb_dasum"); return num(env, d);
    case 6: WGB_OK_OR_THROW(wgb_dnrm2(ctx, n, xd, incx, &d), "wgb_dnrm2"); return num(env, d);
    default: WGB_OK_OR_THROW(wgb_idamax(ctx, n, xd, incx, &idx), "wgb_idamax"); return num(env, (double)idx);
  }
  return num(env, (double)r);
}

napi_value ModuleInit(napi_env env, napi_value exports) {
  if (wgb_abi_version() != WGB_ABI_VERSION) {
    std::string msg = "wgblas_hip addon: libwgblas_hip implements C ABI version " +
                      std::to_string(wgb_abi_version()) + ", the addon was built for " +
                      std::to_string(WGB_ABI_VERSION) + " (rebuild with `python -m wgblas_amd.build`)";
    napi_throw_error(env, nullptr, msg.c_str());
    return nullptr;
  }
  struct Fn {
    const char *name;
    napi_callback cb;
  } fns[] = {
      {"deviceCount", DeviceCount}, {"init", Init}, {"destroy", Destroy},
      {"deviceName", DeviceName}, {"setTiming", SetTiming}, {"lastTimeMs", LastTimeMs},
      {"synchronize", Synchronize}, {"malloc", Malloc}, {"free", Free},
      {"upload", Upload}, {"download", Download}, {"gemm", Gemm},
      {"ssyrk", Ssyrk}, {"ssyr2k", Ssyr2k}, {"ssymm", Ssymm},
      {"tri", Tri}, {"sgemv", Sgemv}, {"ger", Ger}, {"syr", Syr}, {"symv", Symv}, {"trmv", Trmv}, {"reduce", Reduce},
  };
  for (const Fn &f : fns) {
    napi_value v;
    if (napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.cb, nullptr, &v) != napi_ok ||
        napi_set_named_property(env, exports, f.name, v) != napi_ok)
      return nullptr;
  }
  if (napi_add_env_cleanup_hook(env, destroy_live_contexts, nullptr) != napi_ok) return nullptr;
  return exports;
}

}  // namespace

NAPI_MODULE(wgblas_hip, ModuleInit)
