// TypeScript declarations for idamax (src/idamax.mjs).
import { HipDevice } from "./init.mjs";
import { GpuVector } from "./classes/GpuVector.mjs";
import type { Timed } from "./types.mjs";

/** The 0-based index of the first largest |x_i| (NaN skipped); -1 when n <= 0. The vectors are all host arrays or all GpuVectors. */
export declare function idamax(
  device: HipDevice,
  n: number,
  x: Float64Array | GpuVector,
  incx: number,
): Promise<{ index: number } & Timed>;
