// Context, device memory, timing and seeded-input generation for libwgblas_hip.
//
// The context stands in for wgblas's GPUDevice (src/init.mjs:31-108): one HIP
// device, one non-blocking stream at default priority on which every routine
// is ordered, and a pair of events for the optional per-call GPU timing that
// wgblas exposes as `gpuTimeMs` (src/util/benchmark.mjs:14-103).
#include "common.h"

#include <cmath>
#include <cstring>
#include <new>

namespace wgb {

static thread_local std::string t_last_error;

int fail(int status, const std::string &msg) {
  t_last_error = msg;
  return status;
}

int fail_hip(hipError_t err, const char *what) {
  t_last_error = std::string(what) + ": " + hipGetErrorString(err);
  return WGB_ERR_HIP;
}

int enter(wgb_ctx *ctx) {
  if (!ctx) return fail(WGB_ERR_NOT_INITIALIZED, "context is null (call wgb_init first)");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return fail_hip(e, "hipSetDevice");
  return WGB_OK;
}

void timing_begin(wgb_ctx *ctx) {
  if (ctx->timing) (void)hipEventRecord(ctx->ev_start, ctx->stream);
}

void timing_end(wgb_ctx *ctx) {
  if (ctx->timing) {
    (void)hipEventRecord(ctx->ev_stop, ctx->stream);
    ctx->timed_once = true;
  }
}

int ensure_op_workspace(wgb_ctx *ctx, size_t bytes) {
  if (ctx->op_ws_bytes >= bytes) return WGB_OK;
  const size_t round = (size_t)16 << 20;
  bytes = (bytes + round - 1) / round * round;
  WGB_CHECK_HIP(hipStreamSynchronize(ctx->stream));
  if (ctx->op_ws) WGB_CHECK_HIP(hipFree(ctx->op_ws));
  ctx->op_ws = nullptr;
  ctx->op_ws_bytes = 0;
  if (hipMalloc(&ctx->op_ws, bytes) != hipSuccess) {
    (void)hipGetLastError();
    ctx->op_ws = nullptr;
    return fail(WGB_ERR_ALLOC, "hipMalloc of the level-2/3 operand workspace failed");
  }
  ctx->op_ws_bytes = bytes;
  return WGB_OK;
}

}  // namespace wgb

using wgb::fail;

extern "C" const char *wgb_last_error(void) { return wgb::t_last_error.c_str(); }

extern "C" int wgb_abi_version(void) { return WGB_ABI_VERSION; }

extern "C" const char *wgb_status_string(int status) {
  switch (status) {
    case WGB_OK: return "ok";
    case WGB_ERR_INVALID_VALUE: return "invalid value";
    case WGB_ERR_HIP: return "HIP runtime error";
    case WGB_ERR_ALLOC: return "device allocation failed";
    case WGB_ERR_NO_DEVICE: return "no such HIP device";
    case WGB_ERR_NOT_INITIALIZED: return "not initialized";
    default: return "unknown status";
  }
}

extern "C" int wgb_device_count(int *count) {
  if (!count) return fail(WGB_ERR_INVALID_VALUE, "count is null");
  int c = 0;
  hipError_t e = hipGetDeviceCount(&c);
  *count = (e == hipSuccess) ? c : 0;
  return WGB_OK;
}

extern "C" int wgb_init(int device, wgb_ctx **out) {
  if (!out) return fail(WGB_ERR_INVALID_VALUE, "out is null");
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
    return fail(WGB_ERR_NO_DEVICE, "no HIP device is visible");
  if (device < 0 || device >= count)
    return fail(WGB_ERR_NO_DEVICE, "device index " + std::to_string(device) + " out of range (" +
                                       std::to_string(count) + " visible)");
  WGB_CHECK_HIP(hipSetDevice(device));
  wgb_ctx *ctx = new (std::nothrow) wgb_ctx();
  if (!ctx) return fail(WGB_ERR_ALLOC, "host allocation of the context failed");
  ctx->device = device;
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e == hipSuccess) {
    std::snprintf(ctx->arch, sizeof(ctx->arch), "%s", prop.gcnArchName);
    ctx->num_cus = prop.multiProcessorCount;
    // the marketing name can be empty when the driver's id table lacks the
    // part; fall back to the architecture and CU count
    if (prop.name[0])
      std::snprintf(ctx->name, sizeof(ctx->name), "%s", prop.name);
    else
      std::snprintf(ctx->name, sizeof(ctx->name), "AMD %.*s (%d CUs)",
                    (int)std::strcspn(prop.gcnArchName, ":"), prop.gcnArchName,
                    prop.multiProcessorCount);
  }
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreate(&ctx->ev_start);
  if (e == hipSuccess) e = hipEventCreate(&ctx->ev_stop);
  if (e == hipSuccess) e = hipMalloc(&ctx->scratch, wgb::kScratchBytes);
  if (e == hipSuccess) ctx->scratch_bytes = wgb::kScratchBytes;
  if (e == hipSuccess) e = hipHostMalloc(&ctx->host_result, 64, hipHostMallocDefault);
  if (e != hipSuccess) {
    int st = wgb::fail_hip(e, "wgb_init");
    wgb_destroy(ctx);
    return st;
  }
  *out = ctx;
  return WGB_OK;
}

extern "C" int wgb_destroy(wgb_ctx *ctx) {
  if (!ctx) return WGB_OK;
  (void)hipSetDevice(ctx->device);
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  if (ctx->scratch) (void)hipFree(ctx->scratch);
  if (ctx->gemm_ws) (void)hipFree(ctx->gemm_ws);
  if (ctx->op_ws) (void)hipFree(ctx->op_ws);
  if (ctx->host_result) (void)hipHostFree(ctx->host_result);
  if (ctx->ev_start) (void)hipEventDestroy(ctx->ev_start);
  if (ctx->ev_stop) (void)hipEventDestroy(ctx->ev_stop);
  if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
  delete ctx;
  return WGB_OK;
}

extern "C" int wgb_device_name(wgb_ctx *ctx, char *name, size_t name_len, char *arch,
                               size_t arch_len) {
  if (!ctx) return fail(WGB_ERR_NOT_INITIALIZED, "context is null (call wgb_init first)");
  if (name && name_len) std::snprintf(name, name_len, "%s", ctx->name);
  if (arch && arch_len) std::snprintf(arch, arch_len, "%s", ctx->arch);
  return WGB_OK;
}

extern "C" int wgb_set_timing(wgb_ctx *ctx, int enabled) {
  if (!ctx) return fail(WGB_ERR_NOT_INITIALIZED, "context is null (call wgb_init first)");
  ctx->timing = enabled != 0;
  ctx->timed_once = false;
  return WGB_OK;
}

extern "C" int wgb_last_time_ms(wgb_ctx *ctx, float *ms) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if (!ms) return fail(WGB_ERR_INVALID_VALUE, "ms is null");
  if (!ctx->timing || !ctx->timed_once)
    return fail(WGB_ERR_INVALID_VALUE, "no timed call since timing was enabled");
  WGB_CHECK_HIP(hipEventSynchronize(ctx->ev_stop));
  WGB_CHECK_HIP(hipEventElapsedTime(ms, ctx->ev_start, ctx->ev_stop));
  ctx->last_ms = *ms;
  return WGB_OK;
}

extern "C" int wgb_synchronize(wgb_ctx *ctx) {
  int st = wgb::enter(ctx);
  if (st) return st;
  WGB_CHECK_HIP(hipStreamSynchronize(ctx->stream));
  return WGB_OK;
}

extern "C" void *wgb_stream(wgb_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

extern "C" int wgb_malloc(wgb_ctx *ctx, size_t bytes, void **dptr) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if (!dptr) return fail(WGB_ERR_INVALID_VALUE, "dptr is null");
  *dptr = nullptr;
  if (bytes == 0) bytes = 4;  // a zero-length operand still gets a valid handle
  hipError_t e = hipMalloc(dptr, bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(WGB_ERR_ALLOC, "hipMalloc of " + std::to_string(bytes) + " bytes failed: " +
                                   hipGetErrorString(e));
  }
  return WGB_OK;
}

extern "C" int wgb_free(wgb_ctx *ctx, void *dptr) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if (!dptr) return WGB_OK;
  // Work already queued on the stream may still read the buffer.
  WGB_CHECK_HIP(hipStreamSynchronize(ctx->stream));
  WGB_CHECK_HIP(hipFree(dptr));
  return WGB_OK;
}

extern "C" int wgb_memcpy_h2d(wgb_ctx *ctx, void *dst, const void *src, size_t bytes) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if (bytes == 0) return WGB_OK;
  if (!dst || !src) return fail(WGB_ERR_INVALID_VALUE, "null pointer in wgb_memcpy_h2d");
  WGB_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  WGB_CHECK_HIP(hipStreamSynchronize(ctx->stream));
  return WGB_OK;
}

extern "C" int wgb_memcpy_d2h(wgb_ctx *ctx, void *dst, const void *src, size_t bytes) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if (bytes == 0) return WGB_OK;
  if (!dst || !src) return fail(WGB_ERR_INVALID_VALUE, "null pointer in wgb_memcpy_d2h");
  WGB_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  WGB_CHECK_HIP(hipStreamSynchronize(ctx->stream));
  return WGB_OK;
}

extern "C" int wgb_memcpy_d2d(wgb_ctx *ctx, void *dst, const void *src, size_t bytes) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if (bytes == 0) return WGB_OK;
  if (!dst || !src) return fail(WGB_ERR_INVALID_VALUE, "null pointer in wgb_memcpy_d2d");
  WGB_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
  return WGB_OK;
}

// ---- seeded inputs ---------------------------------------------------------
//
// mulberry32 (src/random/random.mjs:4-12) advances its state by a constant
// each draw, so draw i (0-based) hashes state seed + (i+1)*0x6d2b79f5 and the
// whole sequence can be produced in parallel, bit for bit.

namespace {

constexpr uint32_t kMulberryStep = 0x6d2b79f5u;

__device__ __forceinline__ uint32_t mulberry_hash(uint32_t a) {
  uint32_t t = (a ^ (a >> 15)) * (1u | a);
  t = (t + (t ^ (t >> 7)) * (61u | t)) ^ t;
  return t ^ (t >> 14);
}

__device__ __forceinline__ double mulberry_unit(uint32_t seed, uint64_t draw) {
  uint32_t a = seed + (uint32_t)((draw + 1) * (uint64_t)kMulberryStep);
  return (double)mulberry_hash(a) * 0x1p-32;
}

// x[i] = low + next()*(high - low) in double (no contraction: JavaScript
// rounds the product before the sum), then stored in the element type.
template <typename T>
__global__ void fill_uniform_kernel(T *out, int64_t n, double low, double range, uint32_t seed) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    double u = mulberry_unit(seed, (uint64_t)i);
    double v = __dadd_rn(low, __dmul_rn(u, range));
    out[i] = (T)v;
  }
}

__global__ void fill_normal_kernel(float *out, int64_t n, uint32_t seed) {
  int64_t npairs = (n + 1) / 2;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const double two_pi = 6.283185307179586476925286766559;
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < npairs; p += stride) {
    double u1 = mulberry_unit(seed, (uint64_t)(2 * p));
    double u2 = mulberry_unit(seed, (uint64_t)(2 * p + 1));
    double r = sqrt(-2.0 * log(1.0 - u1));
    double t = two_pi * u2;
    double s, c;
    sincos(t, &s, &c);
    out[2 * p] = (float)(r * c);
    if (2 * p + 1 < n) out[2 * p + 1] = (float)(r * s);
  }
}

int fill_grid(int64_t n) {
  int64_t blocks = (n + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  if (blocks < 1) blocks = 1;
  return (int)blocks;
}

}  // namespace

extern "C" int wgb_fill_uniform_f32(wgb_ctx *ctx, float *d_out, int64_t n, double low, double high,
                                    uint32_t seed) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if (n < 0) return fail(WGB_ERR_INVALID_VALUE, "n must be non-negative");
  if (n == 0) return WGB_OK;
  if (!d_out) return fail(WGB_ERR_INVALID_VALUE, "d_out is null");
  fill_uniform_kernel<float><<<fill_grid(n), 256, 0, ctx->stream>>>(d_out, n, low, high - low, seed);
  WGB_CHECK_LAUNCH("fill_uniform_kernel<float>");
  return WGB_OK;
}

extern "C" int wgb_fill_uniform_f64(wgb_ctx *ctx, double *d_out, int64_t n, double low, double high,
                                    uint32_t seed) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if (n < 0) return fail(WGB_ERR_INVALID_VALUE, "n must be non-negative");
  if (n == 0) return WGB_OK;
  if (!d_out) return fail(WGB_ERR_INVALID_VALUE, "d_out is null");
  fill_uniform_kernel<double><<<fill_grid(n), 256, 0, ctx->stream>>>(d_out, n, low, high - low, seed);
  WGB_CHECK_LAUNCH("fill_uniform_kernel<double>");
  return WGB_OK;
}

extern "C" int wgb_fill_normal_f32(wgb_ctx *ctx, float *d_out, int64_t n, uint32_t seed) {
  int st = wgb::enter(ctx);
  if (st) return st;
  if (n < 0) return fail(WGB_ERR_INVALID_VALUE, "n must be non-negative");
  if (n == 0) return WGB_OK;
  if (!d_out) return fail(WGB_ERR_INVALID_VALUE, "d_out is null");
  fill_normal_kernel<<<fill_grid((n + 1) / 2), 256, 0, ctx->stream>>>(d_out, n, seed);
  WGB_CHECK_LAUNCH("fill_normal_kernel");
  return WGB_OK;
}
