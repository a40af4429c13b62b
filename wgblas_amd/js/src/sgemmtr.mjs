// sgemmtr: C <- alpha*op(A)*op(B) + beta*C on the uplo triangle of the
// m x n C only (wgblas src/sgemmtr/sgemmtr.mjs:25-278); the other triangle
// is neither read nor written (wgb_sgemmtr launches only the tiles that meet
// the triangle).
import { checkGemm, runGemm, UPLO } from "./gemm_common.mjs";

export async function sgemmtr(device, uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta,
                              C, ldc, layout = "row-major") {
  const a = { uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, layout };
  const eff = checkGemm(device, a, { routine: "sgemmtr", uplo: true, f64: false });
  if (eff === null) return C instanceof Float32Array ? { C } : {};
  return runGemm(device, 1, a, eff, UPLO[uplo], Float32Array);
}
