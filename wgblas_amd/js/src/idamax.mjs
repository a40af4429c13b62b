// idamax: 0-based logical index of the first max |x[i*incx]| over float64
// values (wgblas src/idamax/idamax.mjs). NaN is never selected, an all-NaN
// vector gives 0, n <= 0 gives -1.
import { reduceOne, shape } from "./level1.mjs";

export async function idamax(device, n, x, incx) {
  return shape("index", reduceOne("idamax", device, n, x, incx, -1));
}
