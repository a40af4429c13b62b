// TypeScript declarations for strmv (src/strmv.mjs).
import { HipDevice } from "./init.mjs";
import { GpuMatrix } from "./classes/GpuMatrix.mjs";
import { GpuVector } from "./classes/GpuVector.mjs";
import type { Diag, Layout, Timed, Trans, Uplo } from "./types.mjs";

/**
 * y = op(A) x, A triangular (x is not modified).
 * Host arrays: `layout` (default row-major) gives their storage order; the
 * result comes back as a new Float32Array under `y` (the input is not modified).
 */
export declare function strmv(
  device: HipDevice,
  uplo: Uplo,
  trans: Trans,
  diag: Diag,
  n: number,
  A: Float32Array,
  lda: number,
  x: Float32Array,
  incx: number,
  y: Float32Array,
  incy: number,
  layout?: Layout,
): Promise<{ y: Float32Array } & Timed>;

/**
 * y = op(A) x, A triangular (x is not modified).
 * Resident operands: each GpuMatrix's own layout applies and `y` is
 * updated in place on the device.
 */
export declare function strmv(
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
