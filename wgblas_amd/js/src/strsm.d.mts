// TypeScript declarations for strsm (src/strsm.mjs).
import { HipDevice } from "./init.mjs";
import { GpuMatrix } from "./classes/GpuMatrix.mjs";
import type { Diag, Layout, Side, Timed, Trans, Uplo } from "./types.mjs";

/**
 * Solves op(A) X = alpha B (side left) or X op(A) = alpha B (right) for X, A triangular; X overwrites B.
 * Host arrays: `layout` (default row-major) gives their storage order; the
 * result comes back as a new Float32Array under `B` (the input is not modified).
 */
export declare function strsm(
  device: HipDevice,
  side: Side,
  uplo: Uplo,
  transA: Trans,
  diag: Diag,
  m: number,
  n: number,
  alpha: number,
  A: Float32Array,
  lda: number,
  B: Float32Array,
  ldb: number,
  layout?: Layout,
): Promise<{ B: Float32Array } & Timed>;

/**
 * Solves op(A) X = alpha B (side left) or X op(A) = alpha B (right) for X, A triangular; X overwrites B.
 * Resident operands: each GpuMatrix's own layout applies and `B` is
 * updated in place on the device.
 */
export declare function strsm(
  device: HipDevice,
  side: Side,
  uplo: Uplo,
  transA: Trans,
  diag: Diag,
  m: number,
  n: number,
  alpha: number,
  A: GpuMatrix,
  lda: number,
  B: GpuMatrix,
  ldb: number,
): Promise<Timed>;
