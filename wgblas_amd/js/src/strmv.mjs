// strmv: y <- op(T) x out of place, T the uplo triangle of A (wgblas
// src/strmv/strmv.mjs:20-259), on wgb_strmv; dtrmv (src/dtrmv/dtrmv.mjs:24-355)
// on wgb_dtrmv through the same function. Argument checks keep wgblas's
// order and messages (strmv.mjs:39-95, dtrmv.mjs); the fp32 routine reads
// a Float64Array-backed resident operand through its float32 rounding, as
// every fp32 routine here does (narrow.mjs). Returns { y } (a new array) for host arrays, {} when y is a
// GpuVector (written in place); plus gpuTimeMs when init({benchmark:true}).
import { trmv } from "./impl/trmv.mjs";

export async function strmv(device, uplo, trans, diag, n, A, lda, x, incx, y, incy, layout = "row-major") {
  return trmv("strmv", device, uplo, trans, diag, n, A, lda, x, incx, y, incy, layout);
}
