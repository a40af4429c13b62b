// The body strmv (src/strmv.mjs) and dtrmv (src/dtrmv.mjs) share: wgblas's
// argument checks in its order, the column-major mapping and the device call.
import { GpuMatrix } from "../classes/GpuMatrix.mjs";
import { GpuVector } from "../classes/GpuVector.mjs";
import { requireGpuDevice, requireSameDevice } from "../device.mjs";
import { checkLayout, checkResidentDtype, checkTrans, checkUplo, execute } from "../gemm_common.mjs";
import { native } from "../native.mjs";
import { columnMajorUplo } from "./syr.mjs";

/** strmv, or dtrmv (routine "dtrmv": Float64Array operands). */
export async function trmv(routine, device, uplo, trans, diag, n, A, lda, x, incx, y, incy,
                           layout = "row-major") {
  const F = routine === "dtrmv" ? Float64Array : Float32Array;
  const FN = F === Float64Array ? "Float64Array" : "Float32Array";
  const xIsGpu = x instanceof GpuVector;
  const yIsGpu = y instanceof GpuVector;
  const AIsGpu = A instanceof GpuMatrix;
  const isUnit = diag === "unit";
  requireGpuDevice(device);
  requireSameDevice(device, routine, { A, x, y });
  checkUplo(uplo);
  checkTrans("trans", trans);
  if (!isUnit && diag !== "non-unit") throw new Error("diag must be 'unit' or 'non-unit'.");
  checkLayout(layout);
  if (!Number.isInteger(n) || !Number.isInteger(incx) || !Number.isInteger(incy) || !Number.isInteger(lda))
    throw new Error("n, incx, incy, and lda must be integers.");
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
  if (xIsGpu && x._buf === y._buf)
    throw new Error("x and y must not reference the same GPU buffer when both are GpuVectors.");
  if (xIsGpu && !AIsGpu) throw new Error("A must be a GpuMatrix when x and y are GpuVectors.");
  if (AIsGpu && !xIsGpu) throw new Error("x and y must be GpuVectors when A is a GpuMatrix.");
  if (AIsGpu && yIsGpu && A._buf === y._buf) throw new Error("A and y must not reference the same GPU buffer.");
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
  // a row-major A read column-major is A^T: uplo and trans both flip
  // (strmv.mjs:97-103)
  const eff = AIsGpu ? A.layout : layout;
  const u = columnMajorUplo(eff, uplo);
  const t = (eff === "column-major") === (trans === "no-transpose") ? 0 : 1;
  return execute(device, [A, x], y, yIsGpu, F, (ctx, p, py) =>
    native().trmv(ctx, u, t, isUnit ? 1 : 0, n, p[0], lda, p[1], incx, py, incy, F === Float64Array), "y");
}
