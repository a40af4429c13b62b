// ssyr2k: C <- alpha*op(A)*op(B)^T + alpha*op(B)*op(A)^T + beta*C on the uplo
// triangle of the n x n C (wgblas src/ssyr2k/ssyr2k.mjs:27-301), on
// wgb_ssyr2k (two triangle launches, the second with beta = 1, as wgblas).
// Argument checks keep wgblas's order and messages (ssyr2k.mjs:45-133).
import { syr2k } from "./impl/syr2k.mjs";

export async function ssyr2k(device, uplo, trans, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                             layout = "row-major") {
  return syr2k("ssyr2k", device, uplo, trans, n, k, alpha, A, lda, B, ldb, beta, C, ldc, layout);
}
