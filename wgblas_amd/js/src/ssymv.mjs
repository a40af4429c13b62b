// ssymv: y <- alpha*S*x + beta*y, S symmetric from A's uplo triangle (wgblas
// src/ssymv/ssymv.mjs:17-216), on wgb_ssymv; dsymv (src/dsymv/dsymv.mjs:25-336)
// on wgb_dsymv through the same function. Argument checks keep wgblas's
// order and messages (ssymv.mjs:33-95, dsymv.mjs:37-111); the fp32 routine
// reads a Float64Array-backed resident operand through its float32
// rounding, as every fp32 routine here does (narrow.mjs). Returns { y } (a new array) for host arrays, {} when y is a
// GpuVector (updated in place); plus gpuTimeMs when init({benchmark:true}).
import { symv } from "./impl/symv.mjs";

export async function ssymv(device, uplo, n, alpha, A, lda, x, incx, beta, y, incy, layout = "row-major") {
  return symv("ssymv", device, uplo, n, alpha, A, lda, x, incx, beta, y, incy, layout);
}
