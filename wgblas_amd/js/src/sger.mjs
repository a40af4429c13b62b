// sger: A <- alpha*x*y^T + A (wgblas src/sger/sger.mjs:17-176), on wgb_sger;
// dger (src/dger/dger.mjs:21-238) on wgb_dger through the same function.
// Argument checks keep wgblas's order and messages (sger.mjs:30-101,
// dger.mjs:34-110), the vectors' checks after the layout swap as there. The
// fp32 routine reads a Float64Array-backed resident operand through its
// float32 rounding, as every fp32 routine here does (narrow.mjs). Returns { A } (a new array) for host arrays, {}
// when A is a GpuMatrix (updated in place); plus gpuTimeMs when
// init({benchmark:true}).
import { ger } from "./impl/ger.mjs";

export async function sger(device, m, n, alpha, x, incx, y, incy, A, lda, layout = "row-major") {
  return ger("sger", device, m, n, alpha, x, incx, y, incy, A, lda, layout);
}
