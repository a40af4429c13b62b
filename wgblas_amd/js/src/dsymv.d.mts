// TypeScript declarations for dsymv (src/dsymv.mjs).
import { HipDevice } from "./init.mjs";
import { GpuMatrix } from "./classes/GpuMatrix.mjs";
import { GpuVector } from "./classes/GpuVector.mjs";
import type { Layout, Timed, Uplo } from "./types.mjs";

/**
 * y = alpha A x + beta y, A symmetric, read from its uplo triangle.
 * Host arrays: `layout` (default row-major) gives their storage order; the
 * result comes back as a new Float64Array under `y` (the input is not modified).
 */
export declare function dsymv(
  device: HipDevice,
  uplo: Uplo,
  n: number,
  alpha: number,
  A: Float64Array,
  lda: number,
  x: Float64Array,
  incx: number,
  beta: number,
  y: Float64Array,
  incy: number,
  layout?: Layout,
): Promise<{ y: Float64Array } & Timed>;

/**
 * y = alpha A x + beta y, A symmetric, read from its uplo triangle.
 * Resident operands: each GpuMatrix's own layout applies and `y` is
 * updated in place on the device.
 */
export declare function dsymv(
  device: HipDevice,
  uplo: Uplo,
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
