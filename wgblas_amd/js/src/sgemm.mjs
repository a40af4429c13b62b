// sgemm: C <- alpha*op(A)*op(B) + beta*C in float32 (wgblas
// src/sgemm/sgemm.mjs:25-269), on the MI355X fp32 MFMA kernel (wgb_sgemm).
// Returns { C } (a new Float32Array) for host arrays, {} when C is a
// GpuMatrix (updated in place); plus gpuTimeMs when init({benchmark:true}).
import { checkGemm, runGemm } from "./gemm_common.mjs";

export async function sgemm(device, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                            layout = "row-major") {
  const a = { transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, layout };
  const eff = checkGemm(device, a, { routine: "sgemm", uplo: false, f64: false });
  if (eff === null) return C instanceof Float32Array ? { C } : {};
  return runGemm(device, 0, a, eff, 0, Float32Array);
}
