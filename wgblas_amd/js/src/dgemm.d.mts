// TypeScript declarations for dgemm (src/dgemm.mjs).
import { HipDevice } from "./init.mjs";
import { GpuMatrix } from "./classes/GpuMatrix.mjs";
import type { Layout, Timed, Trans } from "./types.mjs";

/**
 * C = alpha op(A) op(B) + beta C.
 * Host arrays: `layout` (default row-major) gives their storage order; the
 * result comes back as a new Float64Array under `C` (the input is not modified).
 */
export declare function dgemm(
  device: HipDevice,
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
 * C = alpha op(A) op(B) + beta C.
 * Resident operands: each GpuMatrix's own layout applies and `C` is
 * updated in place on the device.
 */
export declare function dgemm(
  device: HipDevice,
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
