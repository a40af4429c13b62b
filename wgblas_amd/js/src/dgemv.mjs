// dgemv: y <- alpha*op(A)*x + beta*y in native float64 (wgblas
// src/dgemv/dgemv.mjs:23-341, double-double in dgemv_n.wgsl / dgemv_t.wgsl),
// on wgb_dgemv. Checks and messages follow dgemv.mjs:36-124; alpha = 0 with
// beta = 1 returns y untouched without device work (dgemv.mjs:126).
import { gemv } from "./impl/gemv.mjs";

export async function dgemv(device, trans, m, n, alpha, A, lda, x, incx, beta, y, incy,
                            layout = "row-major") {
  return gemv("dgemv", device, trans, m, n, alpha, A, lda, x, incx, beta, y, incy, layout);
}
