// The body ssymv (src/ssymv.mjs) and dsymv (src/dsymv.mjs) share: wgblas's
// argument checks in its order, the column-major mapping and the device call.
import { GpuMatrix } from "../classes/GpuMatrix.mjs";
import { GpuVector } from "../classes/GpuVector.mjs";
import { requireGpuDevice, requireSameDevice } from "../device.mjs";
import { checkLayout, checkResidentDtype, checkScalar, checkUplo, execute } from "../gemm_common.mjs";
import { native } from "../native.mjs";
import { columnMajorUplo } from "./syr.mjs";

/** ssymv, or dsymv (routine "dsymv": Float64Array operands, reference
 * BLAS's alpha = 0, beta = 1 quick return before any device work,
 * dsymv.mjs:116). */
export async function symv(routine, device, uplo, n, alpha, A, lda, x, incx, beta, y, incy,
                           layout = "row-major") {
  const F = routine === "dsymv" ? Float64Array : Float32Array;
  const FN = F === Float64Array ? "Float64Array" : "Float32Array";
  const xIsGpu = x instanceof GpuVector;
  const yIsGpu = y instanceof GpuVector;
  const AIsGpu = A instanceof GpuMatrix;
  requireGpuDevice(device);
  requireSameDevice(device, routine, { A, x, y });
  checkUplo(uplo);
  checkLayout(layout);
  if (!Number.isInteger(n) || !Number.isInteger(incx) || !Number.isInteger(incy) || !Number.isInteger(lda))
    throw new Error("n, incx, incy, and lda must be integers.");
  checkScalar("alpha", alpha);
  checkScalar("beta", beta);
  if (incx <= 0 || incy <= 0) throw new Error("incx and incy must be positive.");
  if (lda < n) throw new Error("lda must be >= n.");
  if (!AIsGpu && !(A instanceof F)) throw new Error(`A must be a ${FN} or GpuMatrix.`);
  checkResidentDtype("A", A, AIsGpu, F);
  if (!xIsGpu && !(x instanceof F)) throw new Error(`x must be a ${FN} or GpuVector.`);
  if (!yIsGpu && !(y instanceof F)) throw new Error(`y must be a ${FN} or GpuVector.`);
  checkResidentDtype("x", x, xIsGpu, F, "GpuVector");
  checkResidentDtype("y", y, yIsGpu, F, "GpuVector");
  if (xIsGpu !== yIsGpu)
    throw new Error(`x and y must be the same type (both ${FN} or both GpuVector).`);
  if (xIsGpu && !AIsGpu) throw new Error("A must be a GpuMatrix when x and y are GpuVectors.");
  if (AIsGpu && !xIsGpu) throw new Error("x and y must be GpuVectors when A is a GpuMatrix.");
  if (xIsGpu && x._buf === y._buf)
    throw new Error("x and y must not reference the same GPU buffer when both are GpuVectors.");
  if (AIsGpu && lda !== A.lda) throw new Error("lda must match A.lda when A is a GpuMatrix.");
  if (AIsGpu && (A.rows < n || A.cols < n)) throw new Error("A is too small for the given n.");
  if (n < 0) throw new Error("n must be non-negative.");
  if (n === 0) return yIsGpu ? {} : { y };
  if (!AIsGpu && A.length < (n - 1) * lda + n)
    throw new Error("A does not have enough elements for the given n and lda.");
  if (x.length < (n - 1) * incx + 1)
    throw new Error("x does not have enough elements for the given n and incx.");
  if (y.length < (n - 1) * incy + 1)
    throw new Error("y does not have enough elements for the given n and incy.");
  if (F === Float64Array && alpha === 0 && beta === 1) return yIsGpu ? {} : { y };
  // the frame's lower triangle is the column-major upper one (ssymv.mjs:96-99)
  const u = columnMajorUplo(AIsGpu ? A.layout : layout, uplo);
  return execute(device, [A, x], y, yIsGpu, F, (ctx, p, py) =>
    native().symv(ctx, u, n, alpha, p[0], lda, p[1], incx, beta, py, incy, F === Float64Array), "y");
}
