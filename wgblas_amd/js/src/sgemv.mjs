// sgemv: y <- alpha*op(A)*x + beta*y (wgblas src/sgemv/sgemv.mjs:19-254), on
// wgb_sgemv; dgemv (src/dgemv/dgemv.mjs:23-341) on wgb_dgemv through the same
// function. Argument checks keep wgblas's order and messages
// (sgemv.mjs:36-121, dgemv.mjs:36-124). Returns { y } (a new array) for host
// arrays, {} when y is a GpuVector (updated in place); plus gpuTimeMs when
// init({benchmark:true}).
import { gemv } from "./impl/gemv.mjs";

export async function sgemv(device, trans, m, n, alpha, A, lda, x, incx, beta, y, incy,
                            layout = "row-major") {
  return gemv("sgemv", device, trans, m, n, alpha, A, lda, x, incx, beta, y, incy, layout);
}
