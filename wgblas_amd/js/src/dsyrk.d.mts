// TypeScript declarations for dsyrk (src/dsyrk.mjs).
import { HipDevice } from "./init.mjs";
import { GpuMatrix } from "./classes/GpuMatrix.mjs";
import type { Layout, Timed, Trans, Uplo } from "./types.mjs";

/**
 * The uplo triangle of C = alpha op(A) op(A)^T + beta C.
 * Host arrays: `layout` (default row-major) gives their storage order; the
 * result comes back as a new Float64Array under `C` (the input is not modified).
 */
export declare function dsyrk(
  device: HipDevice,
  uplo: Uplo,
  trans: Trans,
  n: number,
  k: number,
  alpha: number,
  A: Float64Array,
  lda: number,
  beta: number,
  C: Float64Array,
  ldc: number,
  layout?: Layout,
): Promise<{ C: Float64Array } & Timed>;

/**
 * The uplo triangle of C = alpha op(A) op(A)^T + beta C.
 * Resident operands: each GpuMatrix's own layout applies and `C` is
 * updated in place on the device.
 */
export declare function dsyrk(
  device: HipDevice,
  uplo: Uplo,
  trans: Trans,
  n: number,
  k: number,
  alpha: number,
  A: GpuMatrix,
  lda: number,
  beta: number,
  C: GpuMatrix,
  ldc: number,
): Promise<Timed>;
