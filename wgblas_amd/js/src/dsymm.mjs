// dsymm: C <- alpha*A*B + beta*C (side 'left') or alpha*B*A + beta*C
// ('right'), A symmetric with only its uplo triangle read, in native float64
// (wgblas src/dsymm/dsymm.mjs:26-381: symmetrize.wgsl on both halves, then
// dgemm_small in double-double), on wgb_dsymm. Checks and messages follow
// dsymm.mjs:46-142.
import { symm } from "./impl/symm.mjs";

export async function dsymm(device, side, uplo, m, n, alpha, A, lda, B, ldb, beta, C, ldc,
                            layout = "row-major") {
  return symm("dsymm", device, side, uplo, m, n, alpha, A, lda, B, ldb, beta, C, ldc, layout);
}
