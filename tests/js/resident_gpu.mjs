// GPU checks of the resident-operand API on one context (init() once, no
// second context, no timing events): GpuMatrix / GpuVector from / read /
// destroy (wgblas src/classes/GpuMatrix.mjs:43-207, GpuVector.mjs:41-106),
// routines on resident operands against the same calls on host arrays,
// gpuName (src/init.mjs:133-143), and Float64Array-backed operands in the
// fp32 routines, which wgblas computes on the float32 half of their
// double-double pair (src/util/f64.mjs:33-63). Registered by validation.mjs
// when it runs with --gpu (registerCleanupTest after every other case);
// every expected value below is exact.
import { test, assert, assertEqual } from "./harness.mjs";

const bitsEqual = (a, b) => {
  if (a.length !== b.length || a.constructor !== b.constructor) return false;
  const ua = a instanceof Float64Array ? new BigUint64Array(a.buffer, a.byteOffset, a.length)
    : new Uint32Array(a.buffer, a.byteOffset, a.length);
  const ub = b instanceof Float64Array ? new BigUint64Array(b.buffer, b.byteOffset, b.length)
    : new Uint32Array(b.buffer, b.byteOffset, b.length);
  for (let i = 0; i < ua.length; i++) if (ua[i] !== ub[i]) return false;
  return true;
};

// Small integers: every product and sum below is exact in float32.
const ints = (n, seed, Arr = Float32Array) => {
  const out = new Arr(n);
  let s = seed >>> 0;
  for (let i = 0; i < n; i++) {
    s = (Math.imul(s, 1103515245) + 12345) >>> 0;
    out[i] = ((s >>> 16) % 7) - 3;
  }
  return out;
};

// wgblas's double-double split of one double (src/util/f64.mjs:15, 33-45).
const hiOf = (x) => Math.fround(x);
const loOf = (x) => (Number.isFinite(Math.fround(x)) ? Math.fround(x - Math.fround(x)) : 0);

export function registerResidentTests(wg, device) {
  test("resident: init() with the same options returns the same device", async () => {
    // wgblas keys its devices by their options (src/init.mjs:14-41): a
    // second init() makes no new context
    const again = await wg.init();
    assert(again === device, "init() returned another device");
    assert(again._ctx === device._ctx, "init() made another context");
  });

  test("resident: gpuName names the gfx950 device", async () => {
    const g = wg.gpuName(device);
    assert(typeof g.description === "string" && g.description.length > 0, "description");
    assert(/^gfx950/.test(g.device), `device ${g.device}`);
    const d = wg.gpuName();
    assertEqual(d.device, g.device, "default device");
  });

  test("resident: GpuMatrix / GpuVector round trips (lda padding stripped, doubles kept)", async () => {
    const rm = wg.GpuMatrix.from(device, new Float32Array([1, 2, 99, 3, 4, 99]), 2, 2, 3);
    assert(bitsEqual(await rm.read(), new Float32Array([1, 2, 3, 4])), "row-major read");
    rm.destroy();
    rm.destroy();  // a second destroy is a no-op
    const cm = wg.GpuMatrix.from(device, new Float32Array([1, 2, 3, 99, 4, 5, 6, 99]), 3, 2, 4, "column-major");
    assertEqual(cm.layout, "column-major", "layout");
    assert(bitsEqual(await cm.read(), new Float32Array([1, 2, 3, 4, 5, 6])), "column-major read");
    cm.destroy();
    const d = new Float64Array([Math.PI, -0, 1e300, 5e-324, -Infinity]);
    const dm = wg.GpuMatrix.from(device, d, 1, 5);
    assert(bitsEqual(await dm.read(), d), "Float64Array matrix round trip");
    dm.destroy();
    const v = wg.GpuVector.from(device, d);
    const back = await v.read();
    assert(back instanceof Float64Array && bitsEqual(back, d), "Float64Array vector round trip");
    v.destroy();
    const fv = wg.GpuVector.from(device, new Float32Array([1.5, -2.25]));
    assert(bitsEqual(await fv.read(), new Float32Array([1.5, -2.25])), "Float32Array vector round trip");
    fv.destroy();
  });

  test("resident: sgemm / dgemm on GpuMatrix operands equal the host-array calls", async () => {
    for (const [routine, Arr] of [["sgemm", Float32Array], ["dgemm", Float64Array]]) {
      for (const layout of ["row-major", "column-major"]) {
        const m = 5, n = 7, k = 6, lda = 9, ldb = 10, ldc = 11;
        const rowMajor = layout === "row-major";
        const A = ints((rowMajor ? m : k) * lda, 1, Arr);
        const B = ints((rowMajor ? k : n) * ldb, 2, Arr);
        const C = ints((rowMajor ? m : n) * ldc, 3, Arr);
        const host = await wg[routine](device, "no-transpose", "no-transpose", m, n, k, 2, A, lda, B, ldb, -1, C, ldc, layout);
        const gA = wg.GpuMatrix.from(device, A, m, k, lda, layout);
        const gB = wg.GpuMatrix.from(device, B, k, n, ldb, layout);
        const gC = wg.GpuMatrix.from(device, C, m, n, ldc, layout);
        try {
          const r = await wg[routine](device, "no-transpose", "no-transpose", m, n, k, 2, gA, lda, gB, ldb, -1, gC, ldc, layout);
          assertEqual(Object.keys(r).length, 0, `${routine} resident returns {}`);
          // host result without the ld padding, in the same layout
          const outer = rowMajor ? m : n, inner = rowMajor ? n : m;
          const want = new Arr(outer * inner);
          for (let r2 = 0; r2 < outer; r2++) want.set(host.C.subarray(r2 * ldc, r2 * ldc + inner), r2 * inner);
          assert(bitsEqual(await gC.read(), want), `${routine} ${layout}`);
          assert(bitsEqual(await gA.read(), (() => { const o = new Arr(m * k); const ou = rowMajor ? m : k, in_ = rowMajor ? k : m; for (let i = 0; i < ou; i++) o.set(A.subarray(i * lda, i * lda + in_), i * in_); return o; })()), `${routine} A untouched`);
        } finally {
          gA.destroy();
          gB.destroy();
          gC.destroy();
        }
      }
    }
  });

  test("resident: a GpuMatrix's own layout wins over the layout argument", async () => {
    // A row-major resident A and a column-major resident B, called with
    // layout 'column-major': A is read row-major regardless.
    const m = 3, n = 4, k = 2;
    const A = ints(m * k, 4), B = ints(k * n, 5);
    const gA = wg.GpuMatrix.from(device, A, m, k, k, "row-major");
    const gB = wg.GpuMatrix.from(device, B, k, n, k, "column-major");
    const gC = wg.GpuMatrix.from(device, new Float32Array(m * n), m, n, m, "column-major");
    try {
      await wg.sgemm(device, "no-transpose", "no-transpose", m, n, k, 1, gA, k, gB, k, 0, gC, m, "column-major");
      const want = new Float32Array(m * n);
      for (let j = 0; j < n; j++)
        for (let i = 0; i < m; i++) {
          let s = 0;
          for (let p = 0; p < k; p++) s += A[i * k + p] * B[j * k + p];
          want[j * m + i] = s;
        }
      assert(bitsEqual(await gC.read(), want), "mixed storage orders");
    } finally {
      gA.destroy();
      gB.destroy();
      gC.destroy();
    }
  });

  test("resident: fp32 routines read Float64Array-backed operands through their float32 halves", async () => {
    // sgemm with a Float64Array-backed A and C: the product uses fround(A)
    // and fround(C); C comes back as (float32 result) + (C's old low half).
    const m = 2, n = 2, k = 2;
    const A = new Float64Array([1 + 2 ** -30, 2, 3, 4 - 2 ** -28]);
    const B = new Float32Array([1, -1, 2, 5]);
    const C = new Float64Array([3 + 2 ** -40, -7 + 2 ** -35, 1e-3, 1e300]);
    const gA = wg.GpuMatrix.from(device, A, m, k);
    const gB = wg.GpuMatrix.from(device, B, k, n);
    const gC = wg.GpuMatrix.from(device, C, m, n);
    try {
      await wg.sgemm(device, "no-transpose", "no-transpose", m, n, k, 1, gA, k, gB, n, 1, gC, n);
      const want = new Float64Array(m * n);
      for (let i = 0; i < m; i++)
        for (let j = 0; j < n; j++) {
          let s = 0;
          for (let p = 0; p < k; p++) s += hiOf(A[i * k + p]) * B[p * n + j];
          want[i * n + j] = Math.fround(s + hiOf(C[i * n + j])) + loOf(C[i * n + j]);
        }
      const got = await gC.read();
      assert(got instanceof Float64Array, "C stays Float64Array-backed");
      assert(bitsEqual(got, want), `sgemm f64-backed: got ${Array.from(got)}, want ${Array.from(want)}`);
      assert(bitsEqual(await gA.read(), A), "A's doubles untouched");
    } finally {
      gA.destroy();
      gB.destroy();
      gC.destroy();
    }
    // sdot / sasum / isamax read a Float64Array-backed GpuVector as float32
    const x = new Float64Array([1 + 2 ** -30, -2, 3 + 2 ** -29]);
    const y = new Float32Array([1, 1, 1]);
    const gx = wg.GpuVector.from(device, x);
    const gy = wg.GpuVector.from(device, y);
    const gy64 = wg.GpuVector.from(device, new Float64Array([1, 1, 1]));
    try {
      assertEqual((await wg.sdot(device, 3, gx, 1, gy, 1)).dot, 2, "sdot on fround(x)");
      assertEqual((await wg.sasum(device, 3, gx, 1)).asum, 6, "sasum on fround(x)");
      assertEqual((await wg.isamax(device, 3, gx, 1)).index, 2, "isamax");
      assertEqual((await wg.ddot(device, 3, gx, 1, gy64, 1)).dot, x[0] + x[1] + x[2], "ddot keeps the doubles");
    } finally {
      gx.destroy();
      gy.destroy();
      gy64.destroy();
    }
    // sger writes a Float64Array-backed A: fround(A) + alpha x y^T, plus A's
    // old low halves
    const A2 = new Float64Array([1 + 2 ** -33, 2, -3, 4 + 2 ** -31]);
    const gA2 = wg.GpuMatrix.from(device, A2, 2, 2);
    const gx2 = wg.GpuVector.from(device, new Float32Array([1, 2]));
    const gy2 = wg.GpuVector.from(device, new Float32Array([3, -1]));
    try {
      await wg.sger(device, 2, 2, 1, gx2, 1, gy2, 1, gA2, 2);
      const xv = [1, 2], yv = [3, -1];
      const want = new Float64Array(4);
      for (let i = 0; i < 2; i++)
        for (let j = 0; j < 2; j++)
          want[i * 2 + j] = Math.fround(hiOf(A2[i * 2 + j]) + xv[i] * yv[j]) + loOf(A2[i * 2 + j]);
      assert(bitsEqual(await gA2.read(), want), "sger f64-backed A");
    } finally {
      gA2.destroy();
      gx2.destroy();
      gy2.destroy();
    }
  });
}

// Registered last: cleanup() with no argument releases every device
// (src/init.mjs:110-131); the released device then rejects calls and
// gpuName() has no device to name. A GpuMatrix made before stays safe to
// destroy (a no-op once its device is gone).
export function registerCleanupTest(wg, device) {
  test("cleanup() releases every device", async () => {
    const g = wg.GpuMatrix.from(device, new Float32Array([1, 2, 3, 4]), 2, 2);
    wg.cleanup();
    assert(device._ctx === null, "device still holds its context");
    let threw = false;
    try {
      wg.gpuName();
    } catch (e) {
      threw = /init\(\)/.test(e.message);
    }
    assert(threw, "gpuName() after cleanup()");
    let rejected = false;
    try {
      await wg.sdot(device, 2, new Float32Array([1, 2]), 1, new Float32Array([3, 4]), 1);
    } catch (e) {
      rejected = /released by cleanup/.test(e.message);
    }
    assert(rejected, "a call on the released device");
    g.destroy();
    wg.cleanup();  // nothing left: a no-op
  });
}
