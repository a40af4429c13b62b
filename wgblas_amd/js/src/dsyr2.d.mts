// TypeScript declarations for dsyr2 (src/dsyr2.mjs).
import { HipDevice } from "./init.mjs";
import { GpuMatrix } from "./classes/GpuMatrix.mjs";
import { GpuVector } from "./classes/GpuVector.mjs";
import type { Layout, Timed, Uplo } from "./types.mjs";

/**
 * The uplo triangle of A = alpha (x y^T + y x^T) + A.
 * Host arrays: `layout` (default row-major) gives their storage order; the
 * result comes back as a new Float64Array under `A` (the input is not modified).
 */
export declare function dsyr2(
  device: HipDevice,
  uplo: Uplo,
  n: number,
  alpha: number,
  x: Float64Array,
  incx: number,
  y: Float64Array,
  incy: number,
  A: Float64Array,
  lda: number,
  layout?: Layout,
): Promise<{ A: Float64Array } & Timed>;

/**
 * The uplo triangle of A = alpha (x y^T + y x^T) + A.
 * Resident operands: each GpuMatrix's own layout applies and `A` is
 * updated in place on the device.
 */
export declare function dsyr2(
  device: HipDevice,
  uplo: Uplo,
  n: number,
  alpha: number,
  x: GpuVector,
  incx: number,
  y: GpuVector,
  incy: number,
  A: GpuMatrix,
  lda: number,
): Promise<Timed>;
