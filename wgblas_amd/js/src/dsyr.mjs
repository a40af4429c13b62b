// dsyr: A <- alpha*x*x^T + A on one triangle in native float64 (wgblas
// src/dsyr/dsyr.mjs:21-196, double-double in dsyr.wgsl), on wgb_dsyr.
import { syr } from "./impl/syr.mjs";

export async function dsyr(device, uplo, n, alpha, x, incx, A, lda, layout = "row-major") {
  return syr("dsyr", device, uplo, n, alpha, x, incx, A, lda, layout);
}
