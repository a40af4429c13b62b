// ssymm: C <- alpha*A*B + beta*C (side 'left') or alpha*B*A + beta*C
// ('right'), A symmetric with only its uplo triangle read (wgblas
// src/ssymm/ssymm.mjs:30-318), on wgb_ssymm. Argument checks keep wgblas's
// order and messages (ssymm.mjs:48-134).
import { symm } from "./impl/symm.mjs";

export async function ssymm(device, side, uplo, m, n, alpha, A, lda, B, ldb, beta, C, ldc,
                            layout = "row-major") {
  return symm("ssymm", device, side, uplo, m, n, alpha, A, lda, B, ldb, beta, C, ldc, layout);
}
