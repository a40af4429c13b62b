// Float64Array-backed resident operands given to the fp32 routines.
//
// wgblas keeps a Float64Array GpuMatrix / GpuVector as a double-double pair
// of float32 buffers (hi = Math.fround(x) in `_buf`, lo = Math.fround(x - hi)
// in `_loBuf`, 0 when hi is not finite; src/util/f64.mjs:15, 33-45). Its fp32
// routines do not check the dtype: they bind `_buf`, so they compute on the
// float32 rounding of the doubles, and an output's result goes to `_buf`
// alone; read() then returns hi + lo (src/util/f64.mjs:58-63) — the new
// float32 value plus the old low half.
//
// Here such an operand holds native doubles. For an fp32 routine it is
// rounded into a temporary float32 buffer for the call; an output's doubles
// then become (float32 result) + (old low half), element by element, which
// is what wgblas's read() returns after the same call.
import { GpuVector } from "./classes/GpuVector.mjs";

/** Elements in the operand's allocation (GpuMatrix: outer * lda). */
function storageLength(X) {
  if (X instanceof GpuVector) return X.length;
  const outer = X.layout === "column-major" ? X.cols : X.rows;
  return outer * X.lda;
}

/** Whether an fp32 routine must read X through a float32 copy. */
export function needsNarrowing(X, arrayType) {
  return arrayType === Float32Array && X.dtype === Float64Array;
}

/**
 * Rounds resident operand X's doubles into a new float32 device buffer
 * (pushed on `temps`, which the caller frees) and keeps the low halves.
 * Returns { p, lo, n }.
 */
export function narrowResident(nat, ctx, X, temps) {
  const n = storageLength(X);
  const d = new Float64Array(n);
  if (n > 0) nat.download(ctx, X._buf, d);
  const hi = Float32Array.from(d);
  const lo = new Float32Array(n);
  for (let i = 0; i < n; i++) lo[i] = Number.isFinite(hi[i]) ? Math.fround(d[i] - hi[i]) : 0;
  const p = nat.malloc(ctx, hi.byteLength);
  temps.push(p);
  if (n > 0) nat.upload(ctx, p, hi);
  return { p, lo, n };
}

/** Writes an output's float32 result back into X's doubles as result + lo. */
export function widenResident(nat, ctx, X, w) {
  if (w.n === 0) return;
  const r = new Float32Array(w.n);
  nat.download(ctx, w.p, r);
  const out = new Float64Array(w.n);
  for (let i = 0; i < w.n; i++) out[i] = r[i] + w.lo[i];
  nat.upload(ctx, X._buf, out);
}
