// TypeScript declarations for dgemmtr (src/dgemmtr.mjs).
import { HipDevice } from "./init.mjs";
import { GpuMatrix } from "./classes/GpuMatrix.mjs";
import type { Layout, Timed, Trans, Uplo } from "./types.mjs";

/**
 * The uplo triangle of C = alpha op(A) op(B) + beta C; the other triangle is not written.
 * Host arrays: `layout` (default row-major) gives their storage order; the
 * result comes back as a new Float64Array under `C` (the input is not modified).
 */
export declare function dgemmtr(
  device: HipDevice,
  uplo: Uplo,
  transA: Trans,
  transB: Trans,
  m: number,
  n: number,
  k: number,
  alpha: number,
  A: Float64Array,
  lda: number,
  B: Float64Array,
  ldb: number,
  beta: number,
  C: Float64Array,
  ldc: number,
  layout?: Layout,
): Promise<{ C: Float64Array } & Timed>;

/**
 * The uplo triangle of C = alpha op(A) op(B) + beta C; the other triangle is not written.
 * Resident operands: each GpuMatrix's own layout applies and `C` is
 * updated in place on the device.
 */
export declare function dgemmtr(
  device: HipDevice,
  uplo: Uplo,
  transA: Trans,
  transB: Trans,
  m: number,
  n: number,
  k: number,
  alpha: number,
  A: GpuMatrix,
  lda: number,
  B: GpuMatrix,
  ldb: number,
  beta: number,
  C: GpuMatrix,
  ldc: number,
): Promise<Timed>;
