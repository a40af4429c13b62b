// TypeScript declarations for dsyr (src/dsyr.mjs).
import { HipDevice } from "./init.mjs";
import { GpuMatrix } from "./classes/GpuMatrix.mjs";
import { GpuVector } from "./classes/GpuVector.mjs";
import type { Layout, Timed, Uplo } from "./types.mjs";

/**
 * The uplo triangle of A = alpha x x^T + A.
 * Host arrays: `layout` (default row-major) gives their storage order; the
 * result comes back as a new Float64Array under `A` (the input is not modified).
 */
export declare function dsyr(
  device: HipDevice,
  uplo: Uplo,
  n: number,
  alpha: number,
  x: Float64Array,
  incx: number,
  A: Float64Array,
  lda: number,
  layout?: Layout,
): Promise<{ A: Float64Array } & Timed>;

/**
 * The uplo triangle of A = alpha x x^T + A.
 * Resident operands: each GpuMatrix's own layout applies and `A` is
 * updated in place on the device.
 */
export declare function dsyr(
  device: HipDevice,
  uplo: Uplo,
  n: number,
  alpha: number,
  x: GpuVector,
  incx: number,
  A: GpuMatrix,
  lda: number,
): Promise<Timed>;
