// dtrmv: y <- op(T) x in native float64 (wgblas src/dtrmv/dtrmv.mjs:24-355,
// double-double in dtrmv.wgsl, dtrmv_t.wgsl), on wgb_dtrmv.
import { trmv } from "./impl/trmv.mjs";

export async function dtrmv(device, uplo, trans, diag, n, A, lda, x, incx, y, incy, layout = "row-major") {
  return trmv("dtrmv", device, uplo, trans, diag, n, A, lda, x, incx, y, incy, layout);
}
