// dsyr2k: C <- alpha*op(A)*op(B)^T + alpha*op(B)*op(A)^T + beta*C on the
// uplo triangle of the n x n C, in native float64 (wgblas
// src/dsyr2k/dsyr2k.mjs:24-331 runs two dgemm_small passes in
// double-double), on wgb_dsyr2k. Checks and messages follow dsyr2k.mjs:45-145.
import { syr2k } from "./impl/syr2k.mjs";

export async function dsyr2k(device, uplo, trans, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                             layout = "row-major") {
  return syr2k("dsyr2k", device, uplo, trans, n, k, alpha, A, lda, B, ldb, beta, C, ldc, layout);
}
