// isamax: 0-based logical index of the first max |x[i*incx]| (wgblas
// src/isamax/isamax.mjs). NaN is never selected, an all-NaN vector gives 0,
// n <= 0 gives -1.
import { reduceOne, shape } from "./level1.mjs";

export async function isamax(device, n, x, incx) {
  return shape("index", reduceOne("isamax", device, n, x, incx, -1));
}
