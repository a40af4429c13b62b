// TypeScript declarations for dtrmv (src/dtrmv.mjs).
import { HipDevice } from "./init.mjs";
import { GpuMatrix } from "./classes/GpuMatrix.mjs";
import { GpuVector } from "./classes/GpuVector.mjs";
import type { Diag, Layout, Timed, Trans, Uplo } from "./types.mjs";

/**
 * y = op(A) x, A triangular (x is not modified).
 * Host arrays: `layout` (default row-major) gives their storage order; the
 * result comes back as a new Float64Array under `y` (the input is not modified).
 */
export declare function dtrmv(
  device: HipDevice,
  uplo: Uplo,
  trans: Trans,
  diag: Diag,
  n: number,
  A: Float64Array,
  lda: number,
  x: Float64Array,
  incx: number,
  y: Float64Array,
  incy: number,
  layout?: Layout,
): Promise<{ y: Float64Array } & Timed>;

/**
 * y = op(A) x, A triangular (x is not modified).
 * Resident operands: each GpuMatrix's own layout applies and `y` is
 * updated in place on the device.
 */
export declare function dtrmv(
  device: HipDevice,
  uplo: Uplo,
  trans: Trans,
  diag: Diag,
  n: number,
  A: GpuMatrix,
  lda: number,
  x: GpuVector,
  incx: number,
  y: GpuVector,
  incy: number,
): Promise<Timed>;
