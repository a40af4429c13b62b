// The body sgemv (src/sgemv.mjs) and dgemv (src/dgemv.mjs) share: wgblas's
// argument checks in its order, the column-major mapping and the device call.
import { GpuMatrix } from "../classes/GpuMatrix.mjs";
import { GpuVector } from "../classes/GpuVector.mjs";
import { requireGpuDevice, requireSameDevice } from "../device.mjs";
import { checkLayout, checkResidentDtype, checkScalar, checkTrans, execute } from "../gemm_common.mjs";
import { native } from "../native.mjs";

/** sgemv, or dgemv (routine "dgemv": Float64Array operands, reference BLAS's
 * alpha = 0, beta = 1 quick return before any device work,
 * dgemv.mjs:126). */
export async function gemv(routine, device, trans, m, n, alpha, A, lda, x, incx, beta, y, incy,
                           layout = "row-major") {
  const F = routine === "dgemv" ? Float64Array : Float32Array;
  const FN = F === Float64Array ? "Float64Array" : "Float32Array";
  const AIsGpu = A instanceof GpuMatrix;
  const xIsGpu = x instanceof GpuVector;
  const yIsGpu = y instanceof GpuVector;
  requireGpuDevice(device);
  requireSameDevice(device, routine, { A, x, y });
  checkTrans("trans", trans);
  checkLayout(layout);
  checkScalar("alpha", alpha);
  checkScalar("beta", beta);
  for (const v of [m, n, incx, incy, lda])
    if (!Number.isInteger(v)) throw new Error("m, n, incx, incy, and lda must be integers.");
  if (incx <= 0 || incy <= 0) throw new Error("incx and incy must be positive.");
  if (!AIsGpu && !(A instanceof F)) throw new Error(`A must be a ${FN} or GpuMatrix.`);
  if (F === Float64Array) checkResidentDtype("A", A, AIsGpu, F);
  if (!xIsGpu && !(x instanceof F)) throw new Error(`x must be a ${FN} or GpuVector.`);
  if (!yIsGpu && !(y instanceof F)) throw new Error(`y must be a ${FN} or GpuVector.`);
  if (F === Float32Array) checkResidentDtype("A", A, AIsGpu, F);
  checkResidentDtype("x", x, xIsGpu, F, "GpuVector");
  checkResidentDtype("y", y, yIsGpu, F, "GpuVector");
  if (xIsGpu !== yIsGpu)
    throw new Error(`x and y must be the same type (both ${FN} or both GpuVector).`);
  if (xIsGpu && !AIsGpu) throw new Error("A must be a GpuMatrix when x and y are GpuVectors.");
  if (AIsGpu && !xIsGpu) throw new Error("x and y must be GpuVectors when A is a GpuMatrix.");
  if (xIsGpu && x._buf === y._buf)
    throw new Error("x and y must not reference the same GPU buffer when both are GpuVectors.");
  if (AIsGpu && yIsGpu && A._buf === y._buf) throw new Error("A and y must not reference the same GPU buffer.");
  if (AIsGpu && lda !== A.lda) throw new Error("lda must match A.lda when A is a GpuMatrix.");
  if (AIsGpu && (A.rows < m || A.cols < n)) throw new Error("A is too small for the given m and n.");
  if (m < 0 || n < 0) throw new Error("m and n must be non-negative.");
  if (m === 0 || n === 0) return yIsGpu ? {} : { y };
  // wgblas's frame is row-major: a column-major A is A^T row-major
  // (sgemv.mjs:97-101). Its checks run in that frame.
  const effLayout = AIsGpu ? A.layout : layout;
  let [mr, nr, tr] = [m, n, trans];
  if (effLayout === "column-major") [mr, nr, tr] = [n, m, trans === "no-transpose" ? "transpose" : "no-transpose"];
  const isNoTrans = tr === "no-transpose";
  const xLen = isNoTrans ? nr : mr;
  const yLen = isNoTrans ? mr : nr;
  if (lda < nr) throw new Error("lda must be >= n.");
  if (!AIsGpu && A.length < (mr - 1) * lda + nr)
    throw new Error("A does not have enough elements for the given m, n, and lda.");
  if (x.length < (xLen - 1) * incx + 1)
    throw new Error("x does not have enough elements for the given dimensions and incx.");
  if (y.length < (yLen - 1) * incy + 1)
    throw new Error("y does not have enough elements for the given dimensions and incy.");
  // The row-major mr x nr frame matrix read column-major is its nr x mr
  // transpose: op flips.
  // dgemv: reference BLAS's quick return, no device work (dgemv.mjs:126)
  if (F === Float64Array && alpha === 0 && beta === 1) return yIsGpu ? {} : { y };
  const t = isNoTrans ? 1 : 0;
  return execute(device, [A, x], y, yIsGpu, F, (ctx, p, py) =>
    native().sgemv(ctx, t, nr, mr, alpha, p[0], lda, p[1], incx, beta, py, incy, F === Float64Array),
  "y");
}
