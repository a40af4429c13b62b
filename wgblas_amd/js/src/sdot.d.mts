// TypeScript declarations for sdot (src/sdot.mjs).
import { HipDevice } from "./init.mjs";
import { GpuVector } from "./classes/GpuVector.mjs";
import type { Timed } from "./types.mjs";

/** The dot product of x and y, accumulated in fp32. The vectors are all host arrays or all GpuVectors. */
export declare function sdot(
  device: HipDevice,
  n: number,
  x: Float32Array | GpuVector,
  incx: number,
  y: Float32Array | GpuVector,
  incy: number,
): Promise<{ dot: number } & Timed>;
