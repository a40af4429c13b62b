// TypeScript declarations for dasum (src/dasum.mjs).
import { HipDevice } from "./init.mjs";
import { GpuVector } from "./classes/GpuVector.mjs";
import type { Timed } from "./types.mjs";

/** The sum of |x_i|. The vectors are all host arrays or all GpuVectors. */
export declare function dasum(
  device: HipDevice,
  n: number,
  x: Float64Array | GpuVector,
  incx: number,
): Promise<{ asum: number } & Timed>;
