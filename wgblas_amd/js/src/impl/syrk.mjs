// The body ssyrk (src/ssyrk.mjs) and dsyrk (src/dsyrk.mjs) share: wgblas's
// argument checks in its order, the column-major mapping and the device call.
import { GpuMatrix } from "../classes/GpuMatrix.mjs";
import { requireGpuDevice, requireSameDevice } from "../device.mjs";
import {
  checkLayout, checkOperand, checkScalar, checkTrans, checkUplo, execute, TRANS, NO_TRANS, UPLO,
} from "../gemm_common.mjs";
import { native } from "../native.mjs";

/**
 * ssyrk / dsyrk body (routine "ssyrk" or "dsyrk"): wgblas's checks in its
 * order, then the column-major mapping and one device call. dsyrk adds the
 * f64 dtype checks and dgemm's quick return (src/dsyrk/dsyrk.mjs:60-142).
 * Throws synchronously; the async wrappers turn that into a rejection.
 */
export function syrk(routine, device, uplo, trans, n, k, alpha, A, lda, beta, C, ldc, layout) {
  const f64 = routine === "dsyrk";
  const arr = f64 ? Float64Array : Float32Array;
  const arrName = f64 ? "Float64Array" : "Float32Array";
  const AIsGpu = A instanceof GpuMatrix;
  const CIsGpu = C instanceof GpuMatrix;
  requireGpuDevice(device);
  requireSameDevice(device, routine, { A, C });
  checkUplo(uplo);
  checkTrans("trans", trans);
  checkLayout(layout);
  checkScalar("alpha", alpha);
  checkScalar("beta", beta);
  for (const v of [n, k, lda, ldc])
    if (!Number.isInteger(v)) throw new Error("n, k, lda, and ldc must be integers.");
  if (!AIsGpu && !(A instanceof arr)) throw new Error(`A must be a ${arrName} or GpuMatrix.`);
  if (!CIsGpu && !(C instanceof arr)) throw new Error(`C must be a ${arrName} or GpuMatrix.`);
  if (f64 && AIsGpu && A.dtype !== arr) throw new Error(`A must be a ${arrName}-backed GpuMatrix.`);
  if (f64 && CIsGpu && C.dtype !== arr) throw new Error(`C must be a ${arrName}-backed GpuMatrix.`);
  if (AIsGpu && !CIsGpu) throw new Error("C must be a GpuMatrix when A is a GpuMatrix.");
  if (CIsGpu && !AIsGpu) throw new Error("A must be a GpuMatrix when C is a GpuMatrix.");
  if (n < 0 || k < 0) throw new Error("n and k must be non-negative.");
  if (lda <= 0 || ldc <= 0) throw new Error("lda and ldc must be positive.");
  if (n === 0) return CIsGpu ? {} : { C };
  const layoutA = AIsGpu ? A.layout : layout;
  const layoutC = CIsGpu ? C.layout : layout;
  checkOperand(A, AIsGpu, layoutA, trans, n, k, lda, { X: "A", ld: "lda", dims: "n, k, and trans" });
  if (ldc < n) throw new Error("ldc must be >= n.");
  if (CIsGpu) {
    if (ldc !== C.lda) throw new Error("ldc must match C.lda when C is a GpuMatrix.");
    if (C.rows < n || C.cols < n) throw new Error("C is too small for the given n.");
  } else if (C.length < (n - 1) * ldc + n) {
    throw new Error("C does not have enough elements for the given dimensions and ldc.");
  }
  // Column-major frame: a row-major A flips trans; op(A)op(A)^T is
  // symmetric, so a row-major C is the same product stored transposed,
  // i.e. the other triangle.
  const t = (trans === "transpose") !== (layoutA !== "column-major") ? TRANS : NO_TRANS;
  let u = UPLO[uplo];
  if (layoutC !== "column-major") u = u === 1 ? 2 : 1;
  if (f64 && (alpha === 0 || k === 0) && beta === 1) return CIsGpu ? {} : { C };
  return execute(device, [A], C, CIsGpu, arr, (ctx, p, pC) =>
    native().ssyrk(ctx, u, t, n, k, alpha, p[0], lda, beta, pC, ldc, f64),
  );
}
