// strmm: B <- alpha*op(A)*B (side 'left') or alpha*B*op(A) ('right'), A
// triangular (wgblas src/strmm/strmm.mjs:30-344), on wgb_strmm: A's
// triangle is copied with zeros elsewhere and the GEMM runs only the k band
// each tile of the triangle reaches. B is updated in place for a GpuMatrix;
// host arrays come back as a new { B }.
import { runTri } from "./tri_common.mjs";

export async function strmm(device, side, uplo, transA, diag, m, n, alpha, A, lda, B, ldb,
                            layout = "row-major") {
  return runTri(0, "strmm", device, side, uplo, transA, diag, m, n, alpha, A, lda, B, ldb, layout);
}
