// The body ssyr (src/ssyr.mjs) and dsyr (src/dsyr.mjs) share: wgblas's
// argument checks in its order, the column-major mapping and the device call.
import { GpuMatrix } from "../classes/GpuMatrix.mjs";
import { GpuVector } from "../classes/GpuVector.mjs";
import { requireGpuDevice, requireSameDevice } from "../device.mjs";
import { checkLayout, checkResidentDtype, checkScalar, checkUplo, execute } from "../gemm_common.mjs";
import { native } from "../native.mjs";

/** ssyr, or dsyr (routine "dsyr": Float64Array operands). */
export async function syr(routine, device, uplo, n, alpha, x, incx, A, lda, layout = "row-major") {
  const F = routine === "dsyr" ? Float64Array : Float32Array;
  const FN = F === Float64Array ? "Float64Array" : "Float32Array";
  const xIsGpu = x instanceof GpuVector;
  const AIsGpu = A instanceof GpuMatrix;
  requireGpuDevice(device);
  requireSameDevice(device, routine, { A, x });
  checkUplo(uplo);
  checkLayout(layout);
  if (!Number.isInteger(n) || !Number.isInteger(incx) || !Number.isInteger(lda))
    throw new Error("n, incx, and lda must be integers.");
  checkScalar("alpha", alpha);
  if (incx <= 0) throw new Error("incx must be positive.");
  if (lda < n) throw new Error("lda must be >= n.");
  if (!AIsGpu && !(A instanceof F)) throw new Error(`A must be a ${FN} or GpuMatrix.`);
  checkResidentDtype("A", A, AIsGpu, F);
  if (!xIsGpu && !(x instanceof F)) throw new Error(`x must be a ${FN} or GpuVector.`);
  checkResidentDtype("x", x, xIsGpu, F, "GpuVector");
  if (xIsGpu && !AIsGpu) throw new Error("A must be a GpuMatrix when x is a GpuVector.");
  if (AIsGpu && !xIsGpu) throw new Error("x must be a GpuVector when A is a GpuMatrix.");
  if (AIsGpu && xIsGpu && A._buf === x._buf) throw new Error("A and x must not reference the same GPU buffer.");
  if (AIsGpu && lda !== A.lda) throw new Error("lda must match A.lda when A is a GpuMatrix.");
  if (AIsGpu && (A.rows < n || A.cols < n)) throw new Error("A is too small for the given n.");
  if (n < 0) throw new Error("n must be non-negative.");
  if (n === 0) return AIsGpu ? {} : { A };
  if (!AIsGpu && A.length < (n - 1) * lda + n)
    throw new Error("A does not have enough elements for the given n and lda.");
  if (x.length < (n - 1) * incx + 1)
    throw new Error("x does not have enough elements for the given n and incx.");
  // reference BLAS quick return: A as it is, x unread (ssyr.mjs:75)
  if (alpha === 0) return AIsGpu ? {} : { A };
  // wgblas's frame is row-major: its lower triangle is the column-major
  // upper one (ssyr.mjs:68-71)
  const u = columnMajorUplo(AIsGpu ? A.layout : layout, uplo);
  return execute(device, [x], A, AIsGpu, F, (ctx, p, pA) =>
    native().syr(ctx, u, n, alpha, p[0], incx, null, 1, pA, lda, F === Float64Array), "A");
}

/** WGB_LOWER (1) / WGB_UPPER (2) of the column-major C ABI for a symmetric
 * A stored in `layout` with wgblas's `uplo`. */
export function columnMajorUplo(layout, uplo) {
  const lower = layout === "column-major" ? uplo === "lower" : uplo === "upper";
  return lower ? 1 : 2;
}
