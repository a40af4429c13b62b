// ssyrk: C <- alpha*op(A)*op(A)^T + beta*C on the uplo triangle of the
// n x n C (wgblas src/ssyrk/ssyrk.mjs:28-244). wgblas copies A into a
// second buffer to bind it as B; wgb_ssyrk reads A once for both operands.
// Argument checks keep wgblas's order and messages (ssyrk.mjs:45-108).
import { syrk } from "./impl/syrk.mjs";

export async function ssyrk(device, uplo, trans, n, k, alpha, A, lda, beta, C, ldc,
                            layout = "row-major") {
  return syrk("ssyrk", device, uplo, trans, n, k, alpha, A, lda, beta, C, ldc, layout);
}
