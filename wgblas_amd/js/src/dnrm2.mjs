// dnrm2: overflow-safe Euclidean norm in native float64 (wgblas
// src/dnrm2/dnrm2.mjs runs Blue's algorithm in double-double with thresholds
// moved into f32's exponent range; wgb_dnrm2 uses LAPACK 3.10's dnrm2
// thresholds for IEEE double). NaN gives NaN, Inf gives Inf, n <= 0 gives 0.
import { reduceOne, shape } from "./level1.mjs";

export async function dnrm2(device, n, x, incx) {
  return shape("nrm2", reduceOne("dnrm2", device, n, x, incx, 0));
}
