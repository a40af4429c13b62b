// ddot: sum of x[i*incx]*y[i*incy] in native float64 (wgblas
// src/ddot/ddot.mjs computes it in double-double), on wgb_ddot's two-pass
// device reduction. n <= 0 gives 0.
import { reduceDot, shape } from "./level1.mjs";

export async function ddot(device, n, x, incx, y, incy) {
  return shape("dot", reduceDot(device, n, x, incx, y, incy, "ddot"));
}
