// Shared checks and execution of the level-1 reductions, in wgblas's order
// and with its messages (src/sdot/sdot.mjs:22-48, src/sasum/sasum.mjs,
// src/snrm2/snrm2.mjs:21-31, src/isamax/isamax.mjs:21-34; the fp64 routines
// add the Float64Array-backed GpuVector checks: src/ddot/ddot.mjs:23-52,
// src/dasum/dasum.mjs:21-35, src/dnrm2/dnrm2.mjs:26-40,
// src/idamax/idamax.mjs:21-37).
import { GpuVector } from "./classes/GpuVector.mjs";
import { requireGpuDevice, requireSameDevice } from "./device.mjs";
import { lastGpuTimeMs } from "./init.mjs";
import { native } from "./native.mjs";
import { narrowResident, needsNarrowing } from "./narrow.mjs";

export const KIND = { sdot: 0, sasum: 1, snrm2: 2, isamax: 3, ddot: 4, dasum: 5, dnrm2: 6, idamax: 7 };

const f64Routine = (routine) => routine[0] === "d" || routine === "idamax";

/** One-vector routines (sasum, snrm2, isamax, dasum, dnrm2, idamax). */
export function reduceOne(routine, device, n, x, incx, emptyValue) {
  const f64 = f64Routine(routine);
  const arrName = f64 ? "Float64Array" : "Float32Array";
  const xIsGpu = x instanceof GpuVector;
  requireGpuDevice(device);
  requireSameDevice(device, routine, { x });
  if (!Number.isInteger(n) || !Number.isInteger(incx)) throw new Error("n and incx must be integers.");
  if (incx <= 0) throw new Error("incx must be positive.");
  if (!xIsGpu && !(x instanceof (f64 ? Float64Array : Float32Array)))
    throw new Error(`x must be a ${arrName} or GpuVector.`);
  if (f64 && xIsGpu && x.dtype !== Float64Array) throw new Error(`x must be a ${arrName}-backed GpuVector.`);
  if (n <= 0) return { value: emptyValue };
  if (x.length < (n - 1) * incx + 1)
    throw new Error("x does not have enough elements for the given n and incx.");
  return run(device, [x], f64 ? Float64Array : Float32Array,
    (ctx, p) => native().reduce(KIND[routine], ctx, n, p[0], incx));
}

/** The two-vector form (sdot, ddot). */
export function reduceDot(device, n, x, incx, y, incy, routine = "sdot") {
  const f64 = routine === "ddot";
  const Arr = f64 ? Float64Array : Float32Array;
  const arrName = f64 ? "Float64Array" : "Float32Array";
  const xIsGpu = x instanceof GpuVector;
  const yIsGpu = y instanceof GpuVector;
  requireGpuDevice(device);
  requireSameDevice(device, routine, { x, y });
  if (!Number.isInteger(n) || !Number.isInteger(incx) || !Number.isInteger(incy))
    throw new Error("n, incx, and incy must be integers.");
  if (incx <= 0 || incy <= 0) throw new Error("incx and incy must be positive.");
  if (!xIsGpu && !(x instanceof Arr)) throw new Error(`x must be a ${arrName} or GpuVector.`);
  if (!yIsGpu && !(y instanceof Arr)) throw new Error(`y must be a ${arrName} or GpuVector.`);
  if (f64 && xIsGpu && x.dtype !== Arr) throw new Error(`x must be a ${arrName}-backed GpuVector.`);
  if (f64 && yIsGpu && y.dtype !== Arr) throw new Error(`y must be a ${arrName}-backed GpuVector.`);
  if (xIsGpu !== yIsGpu)
    throw new Error(`x and y must be the same type (both ${arrName} or both GpuVector).`);
  if (n <= 0) return { value: 0 };
  if (x.length < (n - 1) * incx + 1)
    throw new Error("x does not have enough elements for the given n and incx.");
  if (y.length < (n - 1) * incy + 1)
    throw new Error("y does not have enough elements for the given n and incy.");
  return run(device, [x, y], Arr,
    (ctx, p) => native().reduce(KIND[routine], ctx, n, p[0], incx, p[1], incy));
}

// Host arrays go to temporary device buffers (freed before returning);
// GpuVectors are read in place, a Float64Array-backed one in an fp32
// routine through its float32 rounding (narrow.mjs: wgblas binds that
// vector's float32 half). The scalar result comes back to the host.
function run(device, vectors, arrayType, call) {
  const nat = native();
  const ctx = device.ctx();
  const temps = [];
  const narrowed = new Map();
  try {
    const ptrs = vectors.map((v) => {
      if (v instanceof GpuVector && needsNarrowing(v, arrayType)) {
        if (!narrowed.has(v)) narrowed.set(v, narrowResident(nat, ctx, v, temps).p);
        return narrowed.get(v);
      }
      if (v instanceof GpuVector) return v._buf;
      const p = nat.malloc(ctx, v.byteLength);
      temps.push(p);
      nat.upload(ctx, p, v);
      return p;
    });
    const value = call(ctx, ptrs);
    return { value, gpuTimeMs: lastGpuTimeMs(device) };
  } finally {
    for (const p of temps) nat.free(ctx, p);
  }
}

/** { [key]: value } plus gpuTimeMs when the device is in benchmark mode. */
export function shape(key, r) {
  const out = {};
  out[key] = r.value;
  if (r.gpuTimeMs !== undefined) out.gpuTimeMs = r.gpuTimeMs;
  return out;
}
