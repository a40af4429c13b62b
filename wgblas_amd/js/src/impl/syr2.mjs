// The body ssyr2 (src/ssyr2.mjs) and dsyr2 (src/dsyr2.mjs) share: wgblas's
// argument checks in its order, the column-major mapping and the device call.
import { GpuMatrix } from "../classes/GpuMatrix.mjs";
import { GpuVector } from "../classes/GpuVector.mjs";
import { requireGpuDevice, requireSameDevice } from "../device.mjs";
import { checkLayout, checkResidentDtype, checkScalar, checkUplo, execute } from "../gemm_common.mjs";
import { native } from "../native.mjs";
import { columnMajorUplo } from "./syr.mjs";

/** ssyr2, or dsyr2 (routine "dsyr2": Float64Array operands). */
export async function syr2(routine, device, uplo, n, alpha, x, incx, y, incy, A, lda,
                           layout = "row-major") {
  const F = routine === "dsyr2" ? Float64Array : Float32Array;
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
  if (AIsGpu && xIsGpu && A._buf === x._buf) throw new Error("A and x must not reference the same GPU buffer.");
  if (AIsGpu && yIsGpu && A._buf === y._buf) throw new Error("A and y must not reference the same GPU buffer.");
  if (xIsGpu && x._buf === y._buf)
    throw new Error("x and y must not reference the same GPU buffer when both are GpuVectors.");
  if (AIsGpu && lda !== A.lda) throw new Error("lda must match A.lda when A is a GpuMatrix.");
  if (AIsGpu && (A.rows < n || A.cols < n)) throw new Error("A is too small for the given n.");
  if (n < 0) throw new Error("n must be non-negative.");
  if (n === 0) return AIsGpu ? {} : { A };
  if (!AIsGpu && A.length < (n - 1) * lda + n)
    throw new Error("A does not have enough elements for the given n and lda.");
  if (x.length < (n - 1) * incx + 1)
    throw new Error("x does not have enough elements for the given n and incx.");
  if (y.length < (n - 1) * incy + 1)
    throw new Error("y does not have enough elements for the given n and incy.");
  // reference BLAS quick return: A as it is, vectors unread (ssyr2.mjs:100)
  if (alpha === 0) return AIsGpu ? {} : { A };
  // the frame's lower triangle is the column-major upper one; x y^T + y x^T
  // is symmetric in x and y, so no swap (ssyr2.mjs:93-96)
  const u = columnMajorUplo(AIsGpu ? A.layout : layout, uplo);
  return execute(device, [x, y], A, AIsGpu, F, (ctx, p, pA) =>
    native().syr(ctx, u, n, alpha, p[0], incx, p[1], incy, pA, lda, F === Float64Array), "A");
}
