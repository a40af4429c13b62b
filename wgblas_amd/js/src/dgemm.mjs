// dgemm: C <- alpha*op(A)*op(B) + beta*C in native float64 (wgblas
// src/dgemm/dgemm.mjs:23-318 computes it in double-double on f32 pairs; here
// it runs on the fp64 MFMA kernel, wgb_dgemm). Keeps wgblas's quick return:
// with (alpha == 0 or k == 0) and beta == 1, C is returned untouched (the
// same object for a host array).
import { checkGemm, runGemm } from "./gemm_common.mjs";

export async function dgemm(device, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                            layout = "row-major") {
  const a = { transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, layout };
  const eff = checkGemm(device, a, { routine: "dgemm", uplo: false, f64: true });
  if (eff === null) return C instanceof Float64Array ? { C } : {};
  if ((alpha === 0 || k === 0) && beta === 1) return eff.CIsGpu ? {} : { C };
  return runGemm(device, 2, a, eff, 0, Float64Array);
}
