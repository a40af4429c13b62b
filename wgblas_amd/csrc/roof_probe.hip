// Re-measures the roofs the kernels are judged against, on the box itself
// (the role of wgblas's benchmarks/roofline/wgblas/bandwidth.js and fma.js):
//   * hbm_read: a chunk-per-block sum over 1 GiB of floats (16-byte loads,
//     several grid sizes and load depths, best kept), the pattern of the
//     level-1 reductions;
//   * hbm_copy: 1 GiB read + 1 GiB written by a grid-stride 16-byte copy;
//   * mfma_f32 / mfma_f64: waves issuing independent v_mfma_f32_16x16x4f32 /
//     v_mfma_f64_16x16x4f64 on register operands (16 / 8 accumulators per
//     wave, no memory traffic in the loop), 1-3 blocks of 4 waves per CU.
// One JSON line per probe on stdout; HIP-event timing.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

namespace {

typedef float F4 __attribute__((ext_vector_type(4)));
typedef double D4 __attribute__((ext_vector_type(4)));

#define PROBE_CHECK(x)                                                                  \
  do {                                                                                  \
    hipError_t e_ = (x);                                                                \
    if (e_ != hipSuccess) {                                                             \
      std::fprintf(stderr, "roof_probe: %s failed: %s\n", #x, hipGetErrorString(e_));   \
      std::exit(1);                                                                     \
    }                                                                                   \
  } while (0)

// Block b sums its contiguous chunk of n4 16-byte vectors, U loads in flight
// per thread; one partial per block.
template <int U, bool NT>
__global__ __launch_bounds__(256) void chunk_sum(const F4 *__restrict__ x, long n4, float *__restrict__ part) {
  const long per = (n4 + gridDim.x - 1) / gridDim.x;
  const long beg = per * blockIdx.x, end = beg + per < n4 ? beg + per : n4;
  F4 acc = F4(0.f);
  long q = beg + threadIdx.x;
  for (; q + (U - 1) * 256 < end; q += U * 256) {
    F4 a[U];
#pragma unroll
    for (int u = 0; u < U; ++u) a[u] = NT ? __builtin_nontemporal_load(&x[q + u * 256]) : x[q + u * 256];
#pragma unroll
    for (int u = 0; u < U; ++u) acc += a[u];
  }
  for (; q < end; q += 256) acc += x[q];
  float v = acc.x + acc.y + acc.z + acc.w;
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  __shared__ float lds[4];
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = lds[0] + lds[1] + lds[2] + lds[3];
}

__global__ __launch_bounds__(256) void copy_kernel(const F4 *__restrict__ a, F4 *__restrict__ b, long n4) {
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) b[i] = a[i];
}

constexpr int kAcc = 16;    // fp32 accumulators per wave (4 registers each)
constexpr int kAcc64 = 8;   // fp64 accumulators per wave (8 registers each)

__global__ __launch_bounds__(256, 2) void mfma_f32(int iters, float a0, float b0, float *out) {
  F4 acc[kAcc];
  for (int i = 0; i < kAcc; ++i) acc[i] = F4(0.f);
  const float a = a0 + threadIdx.x, b = b0 - threadIdx.x;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < kAcc; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[i], 0, 0, 0);
  }
  float s = 0.f;
  for (int i = 0; i < kAcc; ++i) s += acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

__global__ __launch_bounds__(256, 2) void mfma_f64(int iters, double a0, double b0, double *out) {
  D4 acc[kAcc64];
  for (int i = 0; i < kAcc64; ++i) acc[i] = D4(0.0);
  const double a = a0 + threadIdx.x, b = b0 - threadIdx.x;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < kAcc64; ++i) acc[i] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, acc[i], 0, 0, 0);
  }
  double s = 0.0;
  for (int i = 0; i < kAcc64; ++i) s += acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

// Average milliseconds per launch over `reps` launches after two warm-ups.
template <typename L>
float per_launch_ms(L launch, int reps) {
  hipEvent_t a, b;
  PROBE_CHECK(hipEventCreate(&a));
  PROBE_CHECK(hipEventCreate(&b));
  launch();
  launch();
  PROBE_CHECK(hipDeviceSynchronize());
  PROBE_CHECK(hipEventRecord(a));
  for (int i = 0; i < reps; ++i) launch();
  PROBE_CHECK(hipEventRecord(b));
  PROBE_CHECK(hipEventSynchronize(b));
  float ms = 0.f;
  PROBE_CHECK(hipEventElapsedTime(&ms, a, b));
  PROBE_CHECK(hipEventDestroy(a));
  PROBE_CHECK(hipEventDestroy(b));
  return ms / reps;
}

}  // namespace

int main() {
  hipDeviceProp_t prop;
  PROBE_CHECK(hipGetDeviceProperties(&prop, 0));
  const int cus = prop.multiProcessorCount;
  const long n = 1L << 28;  // floats: 1 GiB
  const long n4 = n / 4;
  F4 *x = nullptr, *y = nullptr;
  float *part = nullptr;
  PROBE_CHECK(hipMalloc(&x, n * sizeof(float)));
  PROBE_CHECK(hipMalloc(&y, n * sizeof(float)));
  PROBE_CHECK(hipMalloc(&part, 65536 * sizeof(float)));
  PROBE_CHECK(hipMemset(x, 0, n * sizeof(float)));
  const double bytes = n * 4.0;

  double best = 0.0;
  int best_grid = 0, best_u = 0, best_nt = 0;
  for (int grid : {1024, 2048, 4096, 8192}) {
    for (int variant = 0; variant < 4; ++variant) {
      const float ms = per_launch_ms(
          [&] {
            if (variant == 0) chunk_sum<8, false><<<grid, 256>>>(x, n4, part);
            if (variant == 1) chunk_sum<8, true><<<grid, 256>>>(x, n4, part);
            if (variant == 2) chunk_sum<16, false><<<grid, 256>>>(x, n4, part);
            if (variant == 3) chunk_sum<16, true><<<grid, 256>>>(x, n4, part);
          },
          20);
      const double gbs = bytes / ms / 1e6;
      if (gbs > best) {
        best = gbs;
        best_grid = grid;
        best_u = variant < 2 ? 8 : 16;
        best_nt = variant & 1;
      }
    }
  }
  std::printf("{\"probe\": \"hbm_read\", \"GB/s\": %.1f, \"bytes\": %.0f, \"grid\": %d, \"loads_in_flight\": %d, "
              "\"nontemporal\": %d}\n",
              best, bytes, best_grid, best_u, best_nt);
  std::fflush(stdout);

  double best_copy = 0.0;
  for (int grid : {2048, 4096, 8192, 16384}) {
    const float ms = per_launch_ms([&] { copy_kernel<<<grid, 256>>>(x, y, n4); }, 10);
    const double gbs = 2.0 * bytes / ms / 1e6;
    if (gbs > best_copy) best_copy = gbs;
  }
  std::printf("{\"probe\": \"hbm_copy\", \"GB/s\": %.1f, \"bytes\": %.0f}\n", best_copy, 2.0 * bytes);
  std::fflush(stdout);

  float *outf = nullptr;
  double *outd = nullptr;
  PROBE_CHECK(hipMalloc(&outf, (size_t)cus * 3 * 256 * sizeof(float)));
  PROBE_CHECK(hipMalloc(&outd, (size_t)cus * 3 * 256 * sizeof(double)));
  const int iters = 20000;
  double tf32 = 0.0, tf64 = 0.0;
  for (int bpc = 1; bpc <= 3; ++bpc) {
    const int blocks = cus * bpc;
    // per wave and iteration: one 16x16x4 MFMA (2048 flops) per accumulator
    const double flops32 = (double)blocks * 4 * iters * kAcc * 2048.0;
    const double flops64 = (double)blocks * 4 * iters * kAcc64 * 2048.0;
    const float ms32 = per_launch_ms([&] { mfma_f32<<<blocks, 256>>>(iters, 1.0f, 2.0f, outf); }, 3);
    const float ms64 = per_launch_ms([&] { mfma_f64<<<blocks, 256>>>(iters, 1.0, 2.0, outd); }, 3);
    if (flops32 / ms32 / 1e9 > tf32) tf32 = flops32 / ms32 / 1e9;
    if (flops64 / ms64 / 1e9 > tf64) tf64 = flops64 / ms64 / 1e9;
  }
  std::printf("{\"probe\": \"mfma_f32\", \"TFLOP/s\": %.1f, \"instruction\": \"v_mfma_f32_16x16x4f32\"}\n", tf32);
  std::printf("{\"probe\": \"mfma_f64\", \"TFLOP/s\": %.1f, \"instruction\": \"v_mfma_f64_16x16x4f64\"}\n", tf64);
  std::printf("{\"probe\": \"device\", \"cus\": %d, \"arch\": \"%s\"}\n", cus, prop.gcnArchName);
  std::fflush(stdout);
  PROBE_CHECK(hipFree(x));
  PROBE_CHECK(hipFree(y));
  PROBE_CHECK(hipFree(part));
  PROBE_CHECK(hipFree(outf));
  PROBE_CHECK(hipFree(outd));
  return 0;
}
