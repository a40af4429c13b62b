// The body ssymm (src/ssymm.mjs) and dsymm (src/dsymm.mjs) share: wgblas's
// argument checks in its order, the column-major mapping and the device call.
import { GpuMatrix } from "../classes/GpuMatrix.mjs";
import { requireGpuDevice, requireSameDevice } from "../device.mjs";
import {
  checkLayout, checkOperand, checkResidentDtype, checkScalar, checkUplo, execute, NO_TRANS, TRANS, UPLO,
} from "../gemm_common.mjs";
import { checkSide, SIDE } from "../tri_common.mjs";
import { native } from "../native.mjs";

/** ssymm, or dsymm (routine "dsymm": Float64Array operands, reference
 * BLAS's quick return, wgblas src/dsymm/dsymm.mjs:26-381 with the same
 * checks and messages). */
export async function symm(routine, device, side, uplo, m, n, alpha, A, lda, B, ldb, beta, C, ldc,
                           layout) {
  const F = routine === "dsymm" ? Float64Array : Float32Array;
  const AIsGpu = A instanceof GpuMatrix;
  const BIsGpu = B instanceof GpuMatrix;
  const CIsGpu = C instanceof GpuMatrix;
  requireGpuDevice(device);
  requireSameDevice(device, routine, { A, B, C });
  checkSide(side);
  checkUplo(uplo);
  checkLayout(layout);
  checkScalar("alpha", alpha);
  checkScalar("beta", beta);
  for (const v of [m, n, lda, ldb, ldc])
    if (!Number.isInteger(v)) throw new Error("m, n, lda, ldb, and ldc must be integers.");
  if (!AIsGpu && !(A instanceof F)) throw new Error(`A must be a ${F.name} or GpuMatrix.`);
  if (!BIsGpu && !(B instanceof F)) throw new Error(`B must be a ${F.name} or GpuMatrix.`);
  if (!CIsGpu && !(C instanceof F)) throw new Error(`C must be a ${F.name} or GpuMatrix.`);
  checkResidentDtype("A", A, AIsGpu, F);
  checkResidentDtype("B", B, BIsGpu, F);
  checkResidentDtype("C", C, CIsGpu, F);
  if ((AIsGpu || BIsGpu) && !CIsGpu) throw new Error("C must be a GpuMatrix when A or B is a GpuMatrix.");
  if (CIsGpu && (!AIsGpu || !BIsGpu)) throw new Error("A and B must be GpuMatrix when C is a GpuMatrix.");
  if (m < 0 || n < 0) throw new Error("m and n must be non-negative.");
  if (m === 0 || n === 0) return CIsGpu ? {} : { C };
  const layoutA = AIsGpu ? A.layout : layout;
  const layoutB = BIsGpu ? B.layout : layout;
  const layoutC = CIsGpu ? C.layout : layout;
  const order = side === "left" ? m : n;
  if (lda < order) throw new Error("lda must be >= " + (side === "left" ? "m" : "n") + ".");
  if (AIsGpu) {
    if (lda !== A.lda) throw new Error("lda must match A.lda when A is a GpuMatrix.");
    if (A.rows < order || A.cols < order) throw new Error("A is too small for the given m/n and side.");
  } else if (A.length < (order - 1) * lda + order) {
    throw new Error("A does not have enough elements for the given dimensions and lda.");
  }
  checkOperand(B, BIsGpu, layoutB, "no-transpose", m, n, ldb, { X: "B", ld: "ldb", dims: "m and n" });
  checkOperand(C, CIsGpu, layoutC, "no-transpose", m, n, ldc, { X: "C", ld: "ldc", dims: "m and n" });
  // Column-major frame: a row-major A stores the other triangle of the same
  // symmetric matrix; a row-major C = S B is the column-major C^T = B^T S.
  // B read in C's frame is op(B): itself when B and C share a storage order,
  // its transpose otherwise (wgblas's effLayoutB, ssymm.mjs:85-87, 149-163).
  let u = UPLO[uplo];
  if (layoutA !== "column-major") u = u === 1 ? 2 : 1;
  let s = SIDE[side];
  let [mm, nn] = [m, n];
  if (layoutC !== "column-major") [s, mm, nn] = [3 - s, n, m];
  const tB = layoutB === layoutC ? NO_TRANS : TRANS;
  // Reference BLAS quick return in fp64 (dsymm.mjs:143-145): C as it is.
  if (F === Float64Array && alpha === 0 && beta === 1) return CIsGpu ? {} : { C };
  return execute(device, [A, B], C, CIsGpu, F, (ctx, p, pC) =>
    native().ssymm(ctx, s, u, tB, mm, nn, alpha, p[0], lda, p[1], ldb, beta, pC, ldc, F === Float64Array),
  );
}
