// strsm: solves op(A)*X = alpha*B (side 'left') or X*op(A) = alpha*B
// ('right') for X, overwriting B; A triangular (wgblas
// src/strsm/strsm.mjs:148-583), on wgb_strsm: substitution on diagonal
// blocks of order <= 64 with GEMM updates in between, no explicit inverse,
// so NaN and Infinity land where substitution puts them for host and
// GPU-resident operands alike. alpha = 0 makes B a literal zero.
import { runTri } from "./tri_common.mjs";

export async function strsm(device, side, uplo, transA, diag, m, n, alpha, A, lda, B, ldb,
                            layout = "row-major") {
  return runTri(1, "strsm", device, side, uplo, transA, diag, m, n, alpha, A, lda, B, ldb, layout);
}
