// dsyr2: A <- alpha*x*y^T + alpha*y*x^T + A on one triangle in native float64
// (wgblas src/dsyr2/dsyr2.mjs:21-260, double-double in dsyr2.wgsl), on
// wgb_dsyr2.
import { syr2 } from "./impl/syr2.mjs";

export async function dsyr2(device, uplo, n, alpha, x, incx, y, incy, A, lda, layout = "row-major") {
  return syr2("dsyr2", device, uplo, n, alpha, x, incx, y, incy, A, lda, layout);
}
