// Shared argument checks, layout mapping and execution for sgemm, sgemmtr
// and dgemm.
//
// The checks run in wgblas's order with wgblas's messages (callers and the
// reference's validation specs match them by substring):
// src/sgemm/sgemm.mjs:46-149, src/sgemmtr/sgemmtr.mjs:47-152,
// src/dgemm/dgemm.mjs:44-169.
//
// Layout mapping: the device library is column-major (BLAS's frame). A
// row-major operand's memory, read column-major, is its transpose, so its
// trans flag flips. A row-major C is computed as the column-major
// C^T = op(B)^T op(A)^T: A and B (with their flipped flags and leading
// dimensions) swap places, m and n swap, and uplo names the other triangle.
import { GpuMatrix } from "./classes/GpuMatrix.mjs";
import { GpuVector } from "./classes/GpuVector.mjs";
import { requireGpuDevice, requireSameDevice } from "./device.mjs";
import { lastGpuTimeMs } from "./init.mjs";
import { native } from "./native.mjs";
import { narrowResident, needsNarrowing, widenResident } from "./narrow.mjs";

export const NO_TRANS = 0;
export const TRANS = 1;
export const UPLO = { lower: 1, upper: 2 };

export function checkTrans(name, value) {
  if (value !== "no-transpose" && value !== "transpose")
    throw new Error(`${name} must be 'no-transpose' or 'transpose'.`);
}

export function checkLayout(layout) {
  if (layout !== "row-major" && layout !== "column-major")
    throw new Error("layout must be 'row-major' or 'column-major'.");
}

export function checkScalar(name, v) {
  if (typeof v !== "number") throw new Error(`${name} must be a number.`);
  if (Number.isNaN(v)) throw new Error(`${name} must not be NaN.`);
  if (!Number.isFinite(v)) throw new Error(`${name} must be finite.`);
}

/** The fp64 routines' check that a resident operand holds doubles (e.g.
 * src/dsymm/dsymm.mjs:74-79). The fp32 routines check nothing: wgblas binds
 * a Float64Array-backed operand's float32 half, and execute() reads such an
 * operand through its float32 rounding (narrow.mjs). */
export function checkResidentDtype(name, X, isGpu, arr, kind = "GpuMatrix") {
  if (arr === Float64Array && isGpu && X.dtype !== arr)
    throw new Error(`${name} must be a ${arr.name}-backed ${kind}.`);
}

export function checkUplo(uplo) {
  if (uplo !== "lower" && uplo !== "upper") throw new Error("uplo must be 'lower' or 'upper'.");
}

/**
 * Shape check of one operand. op(X) is opRows x opCols; X is stored as
 * op(X) or its transpose (trans) in `layout` with leading dimension `ld`.
 * `names` carries the operand's letter, its ld's name and the dimension
 * names used in the "too small" message.
 */
export function checkOperand(X, isGpu, layout, trans, opRows, opCols, ld, names) {
  const [sr, sc] = trans === "no-transpose" ? [opRows, opCols] : [opCols, opRows];
  const rowMajor = layout !== "column-major";
  const outer = rowMajor ? sr : sc;
  const inner = rowMajor ? sc : sr;
  if (ld < inner)
    throw new Error(`${names.ld} must be >= ${rowMajor ? "cols" : "rows"} of ${names.X} as stored.`);
  if (isGpu) {
    if (ld !== X.lda) throw new Error(`${names.ld} must match ${names.X}.lda when ${names.X} is a GpuMatrix.`);
    if (X.rows < sr || X.cols < sc) throw new Error(`${names.X} is too small for the given ${names.dims}.`);
  } else if (X.length < (outer - 1) * ld + inner) {
    throw new Error(
      `${names.X} does not have enough elements for the given dimensions and ${names.ld}.`,
    );
  }
}

/**
 * Validates a GEMM-family call. Returns null when m or n is 0 (the caller
 * returns at once), else the effective per-operand layouts. opts: { routine,
 * uplo: bool, f64: bool }.
 */
export function checkGemm(device, a, opts) {
  const arr = opts.f64 ? Float64Array : Float32Array;
  const arrName = opts.f64 ? "Float64Array" : "Float32Array";
  const AIsGpu = a.A instanceof GpuMatrix;
  const BIsGpu = a.B instanceof GpuMatrix;
  const CIsGpu = a.C instanceof GpuMatrix;
  requireGpuDevice(device);
  requireSameDevice(device, opts.routine, { A: a.A, B: a.B, C: a.C });
  if (opts.uplo) checkUplo(a.uplo);
  checkTrans("transA", a.transA);
  checkTrans("transB", a.transB);
  checkLayout(a.layout);
  checkScalar("alpha", a.alpha);
  checkScalar("beta", a.beta);
  for (const v of [a.m, a.n, a.k, a.lda, a.ldb, a.ldc])
    if (!Number.isInteger(v)) throw new Error("m, n, k, lda, ldb, and ldc must be integers.");
  for (const [name, X, isGpu] of [["A", a.A, AIsGpu], ["B", a.B, BIsGpu], ["C", a.C, CIsGpu]]) {
    if (!isGpu && !(X instanceof arr)) throw new Error(`${name} must be a ${arrName} or GpuMatrix.`);
  }
  // dgemm / dgemmtr need Float64Array-backed GpuMatrix operands
  // (src/dgemm/dgemm.mjs:73-78); sgemm / sgemmtr read any GpuMatrix through
  // its float32 values (execute()).
  for (const [name, X, isGpu] of [["A", a.A, AIsGpu], ["B", a.B, BIsGpu], ["C", a.C, CIsGpu]])
    checkResidentDtype(name, X, isGpu, arr);
  if ((AIsGpu || BIsGpu) && !CIsGpu) throw new Error("C must be a GpuMatrix when A or B is a GpuMatrix.");
  if (CIsGpu && (!AIsGpu || !BIsGpu)) throw new Error("A and B must be GpuMatrix when C is a GpuMatrix.");
  if (a.m < 0 || a.n < 0 || a.k < 0) throw new Error("m, n, and k must be non-negative.");
  if (a.lda <= 0 || a.ldb <= 0 || a.ldc <= 0) throw new Error("lda, ldb, and ldc must be positive.");
  if (a.m === 0 || a.n === 0) return null;
  // A GpuMatrix's own layout wins over the `layout` argument.
  const layoutA = AIsGpu ? a.A.layout : a.layout;
  const layoutB = BIsGpu ? a.B.layout : a.layout;
  const layoutC = CIsGpu ? a.C.layout : a.layout;
  checkOperand(a.A, AIsGpu, layoutA, a.transA, a.m, a.k, a.lda, { X: "A", ld: "lda", dims: "m, k, and transA" });
  checkOperand(a.B, BIsGpu, layoutB, a.transB, a.k, a.n, a.ldb, { X: "B", ld: "ldb", dims: "n, k, and transB" });
  checkOperand(a.C, CIsGpu, layoutC, "no-transpose", a.m, a.n, a.ldc, { X: "C", ld: "ldc", dims: "m and n" });
  return { AIsGpu, BIsGpu, CIsGpu, layoutA, layoutB, layoutC };
}

const flipUplo = (u) => (u === 1 ? 2 : u === 2 ? 1 : 0);

/** Maps a validated call onto the column-major device frame. */
export function toColumnMajor(a, eff, uplo) {
  const tA = (a.transA === "transpose") !== (eff.layoutA !== "column-major") ? TRANS : NO_TRANS;
  const tB = (a.transB === "transpose") !== (eff.layoutB !== "column-major") ? TRANS : NO_TRANS;
  if (eff.layoutC === "column-major")
    return { uplo, ta: tA, tb: tB, m: a.m, n: a.n, A: a.A, lda: a.lda, B: a.B, ldb: a.ldb };
  return { uplo: flipUplo(uplo), ta: 1 - tB, tb: 1 - tA, m: a.n, n: a.m, A: a.B, lda: a.ldb, B: a.A, ldb: a.lda };
}

/**
 * Runs one device call. Host-array operands are copied to temporary device
 * buffers (freed before returning) and the output C is read back into a new
 * typed array (the input is not modified), returned under `key` ("C", "B"
 * for strmm / strsm, "y" for sgemv); GpuMatrix / GpuVector operands are used
 * in place, except a Float64Array-backed one in an fp32 routine, which is
 * read through a float32 copy and, as the output, written back as wgblas's
 * read() would return it (narrow.mjs).
 * `launch(ctx, ptrs, ptrC)` issues the call.
 */
export function execute(device, operands, C, CIsGpu, arrayType, launch, key = "C") {
  const nat = native();
  const ctx = device.ctx();
  const temps = [];
  const cache = new Map();
  const narrowed = new Map();
  const upload = (X) => {
    const p = nat.malloc(ctx, X.byteLength);
    temps.push(p);
    nat.upload(ctx, p, X);
    return p;
  };
  const narrowOf = (X) => {
    if (!narrowed.has(X)) narrowed.set(X, narrowResident(nat, ctx, X, temps));
    return narrowed.get(X);
  };
  // Read-only inputs passed as the same array share one upload; C always
  // gets its own buffer, so an input aliasing C is read unmodified.
  const resident = (X) => X instanceof GpuMatrix || X instanceof GpuVector;
  const ptrOf = (X) => {
    if (resident(X)) return needsNarrowing(X, arrayType) ? narrowOf(X).p : X._buf;
    if (!cache.has(X)) cache.set(X, upload(X));
    return cache.get(X);
  };
  try {
    const ptrs = operands.map(ptrOf);
    const pC = resident(C) ? ptrOf(C) : upload(C);
    launch(ctx, ptrs, pC);
    const t = lastGpuTimeMs(device);
    if (CIsGpu && needsNarrowing(C, arrayType)) widenResident(nat, ctx, C, narrowOf(C));
    if (CIsGpu) return t === undefined ? {} : { gpuTimeMs: t };
    const out = new arrayType(C.length);
    nat.download(ctx, pC, out);
    return t === undefined ? { [key]: out } : { [key]: out, gpuTimeMs: t };
  } finally {
    for (const p of temps) nat.free(ctx, p);
  }
}

/** sgemm / sgemmtr / dgemm body after validation (kind 0 / 1 / 2). */
export function runGemm(device, kind, a, eff, uplo, arrayType) {
  const c = toColumnMajor(a, eff, uplo);
  return execute(device, [c.A, c.B], a.C, eff.CIsGpu, arrayType, (ctx, p, pC) =>
    native().gemm(kind, ctx, c.uplo, c.ta, c.tb, c.m, c.n, a.k, a.alpha, p[0], c.lda, p[1], c.ldb,
                  a.beta, pC, a.ldc),
  );
}
