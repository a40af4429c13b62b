// ssyr2: A <- alpha*x*y^T + alpha*y*x^T + A on one triangle (wgblas
// src/ssyr2/ssyr2.mjs:17-184), on wgb_ssyr2; dsyr2 (src/dsyr2/dsyr2.mjs:21-260)
// on wgb_dsyr2 through the same function. Argument checks keep wgblas's
// order and messages (ssyr2.mjs:33-91, dsyr2.mjs:37-103); the fp32 routine
// reads a Float64Array-backed resident operand through its float32 rounding
// (narrow.mjs). Returns { A } for host
// arrays, {} when A is a GpuMatrix; plus gpuTimeMs when
// init({benchmark:true}).
import { syr2 } from "./impl/syr2.mjs";

export async function ssyr2(device, uplo, n, alpha, x, incx, y, incy, A, lda, layout = "row-major") {
  return syr2("ssyr2", device, uplo, n, alpha, x, incx, y, incy, A, lda, layout);
}
