// dtrmm: B <- alpha*op(A)*B (side 'left') or alpha*B*op(A) ('right'), A
// triangular, in native float64 (wgblas src/dtrmm/dtrmm.mjs:28-400:
// triangularize.wgsl on both halves, then dgemm_small), on wgb_dtrmm. B is
// updated in place for a GpuMatrix; host arrays come back as a new { B }.
import { runTri } from "./tri_common.mjs";

export async function dtrmm(device, side, uplo, transA, diag, m, n, alpha, A, lda, B, ldb,
                            layout = "row-major") {
  return runTri(2, "dtrmm", device, side, uplo, transA, diag, m, n, alpha, A, lda, B, ldb, layout);
}
