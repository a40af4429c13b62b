// sdot: sum of x[i*incx]*y[i*incy] in float32 (wgblas src/sdot/sdot.mjs),
// on wgb_sdot's two-pass device reduction. n <= 0 gives 0.
import { reduceDot, shape } from "./level1.mjs";

export async function sdot(device, n, x, incx, y, incy) {
  return shape("dot", reduceDot(device, n, x, incx, y, incy));
}
