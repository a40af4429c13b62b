// The body ssyr2k (src/ssyr2k.mjs) and dsyr2k (src/dsyr2k.mjs) share: wgblas's
// argument checks in its order, the column-major mapping and the device call.
import { GpuMatrix } from "../classes/GpuMatrix.mjs";
import { requireGpuDevice, requireSameDevice } from "../device.mjs";
import {
  checkLayout, checkOperand, checkResidentDtype, checkScalar, checkTrans, checkUplo, execute, TRANS, NO_TRANS,
  UPLO,
} from "../gemm_common.mjs";
import { native } from "../native.mjs";

/** ssyr2k, or dsyr2k (routine "dsyr2k": Float64Array operands, reference
 * BLAS's quick return, wgblas src/dsyr2k/dsyr2k.mjs:24-331 with the same
 * checks and messages). */
export async function syr2k(routine, device, uplo, trans, n, k, alpha, A, lda, B, ldb, beta, C, ldc,
                            layout) {
  const F = routine === "dsyr2k" ? Float64Array : Float32Array;
  const AIsGpu = A instanceof GpuMatrix;
  const BIsGpu = B instanceof GpuMatrix;
  const CIsGpu = C instanceof GpuMatrix;
  requireGpuDevice(device);
  requireSameDevice(device, routine, { A, B, C });
  checkUplo(uplo);
  checkTrans("trans", trans);
  checkLayout(layout);
  checkScalar("alpha", alpha);
  checkScalar("beta", beta);
  for (const v of [n, k, lda, ldb, ldc])
    if (!Number.isInteger(v)) throw new Error("n, k, lda, ldb, and ldc must be integers.");
  if (!AIsGpu && !(A instanceof F)) throw new Error(`A must be a ${F.name} or GpuMatrix.`);
  if (!BIsGpu && !(B instanceof F)) throw new Error(`B must be a ${F.name} or GpuMatrix.`);
  if (!CIsGpu && !(C instanceof F)) throw new Error(`C must be a ${F.name} or GpuMatrix.`);
  checkResidentDtype("A", A, AIsGpu, F);
  checkResidentDtype("B", B, BIsGpu, F);
  checkResidentDtype("C", C, CIsGpu, F);
  if ((AIsGpu || BIsGpu) && !CIsGpu) throw new Error("C must be a GpuMatrix when A or B is a GpuMatrix.");
  if (CIsGpu && (!AIsGpu || !BIsGpu)) throw new Error("A and B must be GpuMatrix when C is a GpuMatrix.");
  if (n < 0 || k < 0) throw new Error("n and k must be non-negative.");
  if (lda <= 0 || ldb <= 0 || ldc <= 0) throw new Error("lda, ldb, and ldc must be positive.");
  if (n === 0) return CIsGpu ? {} : { C };
  const layoutA = AIsGpu ? A.layout : layout;
  const layoutB = BIsGpu ? B.layout : layout;
  const layoutC = CIsGpu ? C.layout : layout;
  checkOperand(A, AIsGpu, layoutA, trans, n, k, lda, { X: "A", ld: "lda", dims: "n, k, and trans" });
  checkOperand(B, BIsGpu, layoutB, trans, n, k, ldb, { X: "B", ld: "ldb", dims: "n, k, and trans" });
  if (ldc < n) throw new Error("ldc must be >= n.");
  if (CIsGpu) {
    if (ldc !== C.lda) throw new Error("ldc must match C.lda when C is a GpuMatrix.");
    if (C.rows < n || C.cols < n) throw new Error("C is too small for the given n.");
  } else if (C.length < (n - 1) * ldc + n) {
    throw new Error("C does not have enough elements for the given dimensions and ldc.");
  }
  // Column-major frame: a row-major operand flips its own trans; the update
  // is symmetric, so a row-major C is the other triangle.
  const tA = (trans === "transpose") !== (layoutA !== "column-major") ? TRANS : NO_TRANS;
  const tB = (trans === "transpose") !== (layoutB !== "column-major") ? TRANS : NO_TRANS;
  let u = UPLO[uplo];
  if (layoutC !== "column-major") u = u === 1 ? 2 : 1;
  // Reference BLAS quick return in fp64 (dsyr2k.mjs:172-174): C as it is.
  if (F === Float64Array && (alpha === 0 || k === 0) && beta === 1) return CIsGpu ? {} : { C };
  // A and B of different storage orders (GpuMatrix operands) get different
  // flags: one native call either way (one gpuTimeMs span).
  return execute(device, [A, B], C, CIsGpu, F, (ctx, p, pC) =>
    native().ssyr2k(ctx, u, tA, tB, n, k, alpha, p[0], lda, p[1], ldb, beta, pC, ldc, F === Float64Array),
  );
}
