// dsyrk: C <- alpha*op(A)*op(A)^T + beta*C on the uplo triangle of the n x n
// C, in native float64 (wgblas src/dsyrk/dsyrk.mjs:28-305 runs dgemm_small
// in double-double with A copied into a second buffer; wgb_dsyrk reads A
// once for both operands). Checks and messages follow dsyrk.mjs:45-119.
import { syrk } from "./impl/syrk.mjs";

export async function dsyrk(device, uplo, trans, n, k, alpha, A, lda, beta, C, ldc,
                            layout = "row-major") {
  return syrk("dsyrk", device, uplo, trans, n, k, alpha, A, lda, beta, C, ldc, layout);
}
