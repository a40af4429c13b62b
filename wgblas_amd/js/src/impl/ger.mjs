// The body sger (src/sger.mjs) and dger (src/dger.mjs) share: wgblas's
// argument checks in its order, the column-major mapping and the device call.
import { GpuMatrix } from "../classes/GpuMatrix.mjs";
import { GpuVector } from "../classes/GpuVector.mjs";
import { requireGpuDevice, requireSameDevice } from "../device.mjs";
import { checkLayout, checkResidentDtype, checkScalar, execute } from "../gemm_common.mjs";
import { native } from "../native.mjs";

/** sger, or dger (routine "dger": Float64Array operands). */
export async function ger(routine, device, m, n, alpha, x, incx, y, incy, A, lda,
                          layout = "row-major") {
  const F = routine === "dger" ? Float64Array : Float32Array;
  const FN = F === Float64Array ? "Float64Array" : "Float32Array";
  const AIsGpu = A instanceof GpuMatrix;
  requireGpuDevice(device);
  requireSameDevice(device, routine, { A, x, y });
  checkLayout(layout);
  checkScalar("alpha", alpha);
  for (const v of [m, n, incx, incy, lda])
    if (!Number.isInteger(v)) throw new Error("m, n, incx, incy, and lda must be integers.");
  if (incx <= 0 || incy <= 0) throw new Error("incx and incy must be positive.");
  if (!AIsGpu && !(A instanceof F)) throw new Error(`A must be a ${FN} or GpuMatrix.`);
  checkResidentDtype("A", A, AIsGpu, F);
  if (AIsGpu && lda !== A.lda) throw new Error("lda must match A.lda when A is a GpuMatrix.");
  if (AIsGpu && (A.rows < m || A.cols < n)) throw new Error("A is too small for the given m and n.");
  // wgblas's frame is row-major: a column-major A is A^T there, whose rank-1
  // update swaps the vectors (sger.mjs:56-64)
  const effLayout = AIsGpu ? A.layout : layout;
  if (effLayout === "column-major") {
    [m, n] = [n, m];
    [x, y] = [y, x];
    [incx, incy] = [incy, incx];
  }
  const xIsGpu = x instanceof GpuVector;
  const yIsGpu = y instanceof GpuVector;
  if (lda < n) throw new Error("lda must be >= n.");
  if (!xIsGpu && !(x instanceof F)) throw new Error(`x must be a ${FN} or GpuVector.`);
  if (!yIsGpu && !(y instanceof F)) throw new Error(`y must be a ${FN} or GpuVector.`);
  checkResidentDtype("x", x, xIsGpu, F, "GpuVector");
  checkResidentDtype("y", y, yIsGpu, F, "GpuVector");
  if (xIsGpu !== yIsGpu)
    throw new Error(`x and y must be the same type (both ${FN} or both GpuVector).`);
  if (xIsGpu && !AIsGpu) throw new Error("A must be a GpuMatrix when x and y are GpuVectors.");
  if (AIsGpu && !xIsGpu) throw new Error("x and y must be GpuVectors when A is a GpuMatrix.");
  if (AIsGpu && xIsGpu && A._buf === x._buf) throw new Error("A and x must not reference the same GPU buffer.");
  if (AIsGpu && yIsGpu && A._buf === y._buf) throw new Error("A and y must not reference the same GPU buffer.");
  if (m < 0 || n < 0) throw new Error("m and n must be non-negative.");
  if (m === 0 || n === 0) return AIsGpu ? {} : { A };
  if (!AIsGpu && A.length < (m - 1) * lda + n)
    throw new Error("A does not have enough elements for the given m, n, and lda.");
  if (x.length < (m - 1) * incx + 1)
    throw new Error("x does not have enough elements for the given m and incx.");
  if (y.length < (n - 1) * incy + 1)
    throw new Error("y does not have enough elements for the given n and incy.");
  // reference BLAS quick return: A as it is, x and y unread (sger.mjs:103)
  if (alpha === 0) return AIsGpu ? {} : { A };
  // The row-major m x n frame read column-major is its n x m transpose:
  // A^T += alpha y x^T (column j of it skipped where x[j] is zero, the
  // frame's row skip of sger.wgsl:38-44).
  return execute(device, [x, y], A, AIsGpu, F, (ctx, p, pA) =>
    native().ger(ctx, n, m, alpha, p[1], incy, p[0], incx, pA, lda, F === Float64Array), "A");
}
