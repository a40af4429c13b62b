// dger: A <- alpha*x*y^T + A in native float64 (wgblas src/dger/dger.mjs:21-238,
// double-double in dger.wgsl), on wgb_dger. Checks and messages follow
// dger.mjs:34-110; alpha = 0 returns A untouched without device work
// (dger.mjs:113).
import { ger } from "./impl/ger.mjs";

export async function dger(device, m, n, alpha, x, incx, y, incy, A, lda, layout = "row-major") {
  return ger("dger", device, m, n, alpha, x, incx, y, incy, A, lda, layout);
}
