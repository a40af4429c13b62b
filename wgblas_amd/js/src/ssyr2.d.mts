// TypeScript declarations for ssyr2 (src/ssyr2.mjs).
import { HipDevice } from "./init.mjs";
import { GpuMatrix } from "./classes/GpuMatrix.mjs";
import { GpuVector } from "./classes/GpuVector.mjs";
import type { Layout, Timed, Uplo } from "./types.mjs";

/**
 * The uplo triangle of A = alpha (x y^T + y x^T) + A.
 * Host arrays: `layout` (default row-major) gives their storage order; the
 * result comes back as a new Float32Array under `A` (the input is not modified).
 */
export declare function ssyr2(
  device: HipDevice,
  uplo: Uplo,
  n: number,
  alpha: number,
  x: Float32Array,
  incx: number,
  y: Float32Array,
  incy: number,
  A: Float32Array,
  lda: number,
  layout?: Layout,
): Promise<{ A: Float32Array } & Timed>;

/**
 * The uplo triangle of A = alpha (x y^T + y x^T) + A.
 * Resident operands: each GpuMatrix's own layout applies and `A` is
 * updated in place on the device.
 */
export declare function ssyr2(
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
