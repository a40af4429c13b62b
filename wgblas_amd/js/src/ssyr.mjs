// ssyr: A <- alpha*x*x^T + A on one triangle (wgblas src/ssyr/ssyr.mjs:17-143),
// on wgb_ssyr; dsyr (src/dsyr/dsyr.mjs:21-196) on wgb_dsyr through the same
// function. Argument checks keep wgblas's order and messages (ssyr.mjs:29-66,
// dsyr.mjs:33-78). The fp32 routine reads a Float64Array-backed resident
// operand through its float32 rounding, as every fp32 routine here does
// (narrow.mjs). Returns { A } (a new array) for
// host arrays, {} when A is a GpuMatrix (updated in place); plus gpuTimeMs
// when init({benchmark:true}).
import { syr } from "./impl/syr.mjs";

export async function ssyr(device, uplo, n, alpha, x, incx, A, lda, layout = "row-major") {
  return syr("ssyr", device, uplo, n, alpha, x, incx, A, lda, layout);
}
