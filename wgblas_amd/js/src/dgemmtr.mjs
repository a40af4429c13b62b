// dgemmtr: C <- alpha*op(A)*op(B) + beta*C on the uplo triangle of the
// m x n C, in native float64 (wgblas src/dgemmtr/dgemmtr.mjs:25-328 computes
// it in double-double with dgemm_small's triangle mask). Same checks and
// messages as dgemm plus uplo, and dgemm's quick return: with (alpha == 0 or
// k == 0) and beta == 1, C is returned untouched (dgemmtr.mjs:189).
import { checkGemm, runGemm, UPLO } from "./gemm_common.mjs";

export async function dgemmtr(device, uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta,
                              C, ldc, layout = "row-major") {
  const a = { uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, layout };
  const eff = checkGemm(device, a, { routine: "dgemmtr", uplo: true, f64: true });
  if (eff === null) return C instanceof Float64Array ? { C } : {};
  if ((alpha === 0 || k === 0) && beta === 1) return eff.CIsGpu ? {} : { C };
  return runGemm(device, 3, a, eff, UPLO[uplo], Float64Array);
}
