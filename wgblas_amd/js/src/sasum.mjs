// sasum: sum of |x[i*incx]| (wgblas src/sasum/sasum.mjs). n <= 0 gives 0.
import { reduceOne, shape } from "./level1.mjs";

export async function sasum(device, n, x, incx) {
  return shape("asum", reduceOne("sasum", device, n, x, incx, 0));
}
