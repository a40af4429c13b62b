// The fixed device workspace of wgb_sgemm_noalloc (gemm.hip), the
// allocation-free sgemm: its split-k partials go to `scratch` instead of the
// context's workspace that wgb_sgemm grows with hipMalloc.
//
// A split tail holds at most one round of tiles (rem * S <= slots), so with
// 128 x 128 fp32 tiles at two blocks per CU on 256 CUs it needs at most
// 512 * 64 KiB = 32 MiB: that is the array's size. Every GPU holds its own
// copy until the process ends, shared by every call on that GPU.
//
// The array sits in this translation unit alone, so its code object is
// loaded onto a device only when the entry point first runs there: processes
// that never call wgb_sgemm_noalloc never load it. In host code `scratch`
// names a host-side stand-in, never the device address: the address is
// looked up once per device (hipGetSymbolAddress, with that device current)
// on the entry point's first call there, and only that pointer is passed on.
#include "common.h"

#include <mutex>

namespace {

static __device__ __align__(256) float scratch[wgb::kNoallocWsBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {nullptr};

}  // namespace

namespace wgb {

int noalloc_workspace(wgb_ctx *ctx, void **ptr) {
  *ptr = nullptr;
  if (ctx->device < 0 || ctx->device >= kMaxDevices)
    return fail(WGB_ERR_INVALID_VALUE, "device index beyond the allocation-free workspace table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[ctx->device]) {
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      (void)hipGetLastError();
      return fail_hip(e == hipSuccess ? hipErrorInvalidSymbol : e,
                      "hipGetSymbolAddress of the allocation-free GEMM workspace");
    }
    g_scratch_ptr[ctx->device] = p;
  }
  *ptr = g_scratch_ptr[ctx->device];
  return WGB_OK;
}

}  // namespace wgb
