// snrm2: overflow-safe Euclidean norm (wgblas src/snrm2/snrm2.mjs; Blue's
// three accumulators and LAPACK 3.10's combine on the device). n <= 0 gives 0.
import { reduceOne, shape } from "./level1.mjs";

export async function snrm2(device, n, x, incx) {
  return shape("nrm2", reduceOne("snrm2", device, n, x, incx, 0));
}
