// TypeScript declarations for ddot (src/ddot.mjs).
import { HipDevice } from "./init.mjs";
import { GpuVector } from "./classes/GpuVector.mjs";
import type { Timed } from "./types.mjs";

/** The dot product of x and y. The vectors are all host arrays or all GpuVectors. */
export declare function ddot(
  device: HipDevice,
  n: number,
  x: Float64Array | GpuVector,
  incx: number,
  y: Float64Array | GpuVector,
  incy: number,
): Promise<{ dot: number } & Timed>;
