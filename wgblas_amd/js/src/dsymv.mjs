// dsymv: y <- alpha*S*x + beta*y in native float64 (wgblas
// src/dsymv/dsymv.mjs:25-336, double-double in dsymv.wgsl), on wgb_dsymv.
import { symv } from "./impl/symv.mjs";

export async function dsymv(device, uplo, n, alpha, A, lda, x, incx, beta, y, incy, layout = "row-major") {
  return symv("dsymv", device, uplo, n, alpha, A, lda, x, incx, beta, y, incy, layout);
}
