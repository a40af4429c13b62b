// dasum: sum of |x[i*incx]| in native float64 (wgblas src/dasum/dasum.mjs
// computes it in double-double). n <= 0 gives 0.
import { reduceOne, shape } from "./level1.mjs";

export async function dasum(device, n, x, incx) {
  return shape("asum", reduceOne("dasum", device, n, x, incx, 0));
}
