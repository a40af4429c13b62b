// TypeScript declarations for snrm2 (src/snrm2.mjs).
import { HipDevice } from "./init.mjs";
import { GpuVector } from "./classes/GpuVector.mjs";
import type { Timed } from "./types.mjs";

/** The Euclidean norm of x, free of overflow and underflow. The vectors are all host arrays or all GpuVectors. */
export declare function snrm2(
  device: HipDevice,
  n: number,
  x: Float32Array | GpuVector,
  incx: number,
): Promise<{ nrm2: number } & Timed>;
