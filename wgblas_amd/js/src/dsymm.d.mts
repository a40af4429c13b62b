// TypeScript declarations for dsymm (src/dsymm.mjs).
import { HipDevice } from "./init.mjs";
import { GpuMatrix } from "./classes/GpuMatrix.mjs";
import type { Layout, Side, Timed, Uplo } from "./types.mjs";

/**
 * C = alpha A B + beta C (side left) or alpha B A + beta C (right), A symmetric, read from its uplo triangle.
 * Host arrays: `layout` (default row-major) gives their storage order; the
 * result comes back as a new Float64Array under `C` (the input is not modified).
 */
export declare function dsymm(
  device: HipDevice,
  side: Side,
  uplo: Uplo,
  m: number,
  n: number,
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
 * C = alpha A B + beta C (side left) or alpha B A + beta C (right), A symmetric, read from its uplo triangle.
 * Resident operands: each GpuMatrix's own layout applies and `C` is
 * updated in place on the device.
 */
export declare function dsymm(
  device: HipDevice,
  side: Side,
  uplo: Uplo,
  m: number,
  n: number,
  alpha: number,
  A: GpuMatrix,
  lda: number,
  B: GpuMatrix,
  ldb: number,
  beta: number,
  C: GpuMatrix,
  ldc: number,
): Promise<Timed>;
