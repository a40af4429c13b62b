// Shared checks and the column-major mapping of strmm, strsm and dtrmm
// (wgblas src/strmm/strmm.mjs:46-129, src/strsm/strsm.mjs:162-247,
// src/dtrmm/dtrmm.mjs:45-113: the same checks, in the same order, with the
// same messages), and ssymm's side check.
import { GpuMatrix } from "./classes/GpuMatrix.mjs";
import { requireGpuDevice, requireSameDevice } from "./device.mjs";
import {
  checkLayout, checkOperand, checkResidentDtype, checkTrans, checkUplo, execute, UPLO,
} from "./gemm_common.mjs";
import { native } from "./native.mjs";

export const SIDE = { left: 1, right: 2 };

export function checkSide(side) {
  if (side !== "left" && side !== "right") throw new Error("side must be 'left' or 'right'.");
}

/**
 * strmm (kind 0) / strsm (kind 1) / dtrmm (kind 2, Float64Array operands,
 * wgblas src/dtrmm/dtrmm.mjs:28-400 with the same checks): validation, then
 * one device call on the column-major frame. Returns { B } (a new typed
 * array) for host arrays, {} when B is a GpuMatrix (updated in place).
 */
export function runTri(kind, routine, device, side, uplo, transA, diag, m, n, alpha, A, lda, B, ldb,
                       layout) {
  const F = kind === 2 ? Float64Array : Float32Array;
  const AIsGpu = A instanceof GpuMatrix;
  const BIsGpu = B instanceof GpuMatrix;
  const isUnit = diag === "unit";
  requireGpuDevice(device);
  requireSameDevice(device, routine, { A, B });
  checkSide(side);
  checkUplo(uplo);
  checkTrans("transA", transA);
  if (!isUnit && diag !== "non-unit") throw new Error("diag must be 'unit' or 'non-unit'.");
  checkLayout(layout);
  if (typeof alpha !== "number") throw new Error("alpha must be a number.");
  if (Number.isNaN(alpha)) throw new Error("alpha must not be NaN.");
  if (!Number.isFinite(alpha)) throw new Error("alpha must be finite.");
  for (const v of [m, n, lda, ldb])
    if (!Number.isInteger(v)) throw new Error("m, n, lda, and ldb must be integers.");
  if (!AIsGpu && !(A instanceof F)) throw new Error(`A must be a ${F.name} or GpuMatrix.`);
  if (!BIsGpu && !(B instanceof F)) throw new Error(`B must be a ${F.name} or GpuMatrix.`);
  checkResidentDtype("A", A, AIsGpu, F);
  checkResidentDtype("B", B, BIsGpu, F);
  if (AIsGpu !== BIsGpu) throw new Error(`A and B must both be GpuMatrix or both be ${F.name}.`);
  if (m < 0 || n < 0) throw new Error("m and n must be non-negative.");
  if (m === 0 || n === 0) return BIsGpu ? {} : { B };
  const layoutA = AIsGpu ? A.layout : layout;
  const layoutB = BIsGpu ? B.layout : layout;
  const order = side === "left" ? m : n;
  if (lda < order) throw new Error("lda must be >= " + (side === "left" ? "m" : "n") + ".");
  if (AIsGpu) {
    if (lda !== A.lda) throw new Error("lda must match A.lda when A is a GpuMatrix.");
    if (A.rows < order || A.cols < order) throw new Error("A is too small for the given m/n and side.");
  } else if (A.length < (order - 1) * lda + order) {
    throw new Error("A does not have enough elements for the given dimensions and lda.");
  }
  checkOperand(B, BIsGpu, layoutB, "no-transpose", m, n, ldb, { X: "B", ld: "ldb", dims: "m and n" });
  // Column-major frame. A row-major A read column-major is A^T: the other
  // triangle, and op(A) with the other trans flag. A row-major B is B^T:
  // op(A) B = X becomes X^T op(A)^T (side and trans flip, m and n swap).
  const aRow = layoutA !== "column-major";
  const bRow = layoutB !== "column-major";
  let u = UPLO[uplo];
  if (aRow) u = u === 1 ? 2 : 1;
  const t = ((transA === "transpose") !== aRow) !== bRow ? 1 : 0;
  let s = SIDE[side];
  let [mm, nn] = [m, n];
  if (bRow) [s, mm, nn] = [3 - s, n, m];
  return execute(device, [A], B, BIsGpu, F, (ctx, p, pB) =>
    native().tri(kind, ctx, s, u, t, isUnit ? 1 : 0, mm, nn, alpha, p[0], lda, pB, ldb), "B");
}
