// TypeScript declarations for sgemv (src/sgemv.mjs).
import { HipDevice } from "./init.mjs";
import { GpuMatrix } from "./classes/GpuMatrix.mjs";
import { GpuVector } from "./classes/GpuVector.mjs";
import type { Layout, Timed, Trans } from "./types.mjs";

/**
 * y = alpha op(A) x + beta y.
 * Host arrays: `layout` (default row-major) gives their storage order; the
 * result comes back as a new Float32Array under `y` (the input is not modified).
 */
export declare function sgemv(
  device: HipDevice,
  trans: Trans,
  m: number,
  n: number,
  alpha: number,
  A: Float32Array,
  lda: number,
  x: Float32Array,
  incx: number,
  beta: number,
  y: Float32Array,
  incy: number,
  layout?: Layout,
): Promise<{ y: Float32Array } & Timed>;

/**
 * y = alpha op(A) x + beta y.
 * Resident operands: each GpuMatrix's own layout applies and `y` is
 * updated in place on the device.
 */
export declare function sgemv(
  device: HipDevice,
  trans: Trans,
  m: number,
  n: number,
  alpha: number,
  A: GpuMatrix,
  lda: number,
  x: GpuVector,
  incx: number,
  beta: number,
  y: GpuVector,
  incy: number,
): Promise<Timed>;
