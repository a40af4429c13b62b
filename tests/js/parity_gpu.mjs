// The single-context part of the JavaScript API's GPU checks (through the
// Node-API addon and libwgblas_hip): the reference's edge-case fixtures
// (exact), its regression scenarios (forward-error bound of
// tests/sgemm/helpers.js, bit checks of untouched triangles / padding /
// k = 0), the GpuMatrix / GpuVector residency forms and layouts, all on the
// one device the runner hands over with setParityDevice() before the cases
// run. Imported by validation.mjs --gpu and by gpu_api.mjs (which adds the
// device-handling and benchmark-mode cases). The expected values come from a
// plain double-precision triple loop here (exact on the integer-valued
// fixtures); the kernels themselves are held to the CPU oracle by the Python
// suites.
import { readFileSync } from "fs";
import { fileURLToPath } from "url";
import { dirname, join } from "path";
import { test, assert, assertEqual } from "./harness.mjs";
import * as wg from "../../wgblas_amd/js/index.mjs";

const here = dirname(fileURLToPath(import.meta.url));
const fixture = (name) => JSON.parse(readFileSync(join(here, "..", "golden", "edge_cases", `${name}.json`), "utf8"));

let device;

/** The device every case here runs on; set before the cases run. */
export function setParityDevice(d) {
  device = d;
}

// ---------------------------------------------------------------- reference
const opElem = (M, ld, layout, trans, r, c) => {
  const [sr, sc] = trans === "transpose" ? [c, r] : [r, c];
  return layout === "column-major" ? M[sc * ld + sr] : M[sr * ld + sc];
};
const cIndex = (ldc, layout, r, c) => (layout === "column-major" ? c * ldc + r : r * ldc + c);
const inTri = (uplo, r, c) => !uplo || (uplo === "lower" ? c <= r : c >= r);

function refGemm(a) {
  const layout = a.layout || "row-major";
  const out = Float64Array.from(a.C);
  const absdot = new Float64Array(a.C.length);
  for (let i = 0; i < a.m; i++)
    for (let j = 0; j < a.n; j++) {
      if (!inTri(a.uplo, i, j)) continue;
      let s = 0;
      let ab = 0;
      if (a.alpha !== 0)
        for (let p = 0; p < a.k; p++) {
          const prod = opElem(a.A, a.lda, layout, a.transA, i, p) * opElem(a.B, a.ldb, layout, a.transB, p, j);
          s += prod;
          ab += Math.abs(prod);
        }
      const idx = cIndex(a.ldc, layout, i, j);
      out[idx] = (a.alpha === 0 ? 0 : a.alpha * s) + (a.beta === 0 ? 0 : a.beta * a.C[idx]);
      absdot[idx] = ab;
    }
  return { out, absdot };
}

// Forward factor of tests/sgemm/helpers.js (eps 2^-23, (k+1)) or
// tests/dgemm/helpers.js (eps 2^-48, (k+2), 3|beta||C|), plus a bit check of
// everything outside the m x n part / triangle.
function checkGemm(got, a, dd) {
  const layout = a.layout || "row-major";
  const { out, absdot } = refGemm(a);
  const eps = dd ? 2 ** -48 : 2 ** -23;
  let worst = 0;
  const touched = new Uint8Array(a.C.length);
  for (let i = 0; i < a.m; i++)
    for (let j = 0; j < a.n; j++) {
      if (!inTri(a.uplo, i, j)) continue;
      const idx = cIndex(a.ldc, layout, i, j);
      touched[idx] = 1;
      const bound = eps * ((a.k + (dd ? 2 : 1)) * Math.abs(a.alpha) * absdot[idx] + (dd ? 3 : 1) * Math.abs(a.beta) * Math.abs(a.C[idx]));
      const err = Math.abs(got[idx] - out[idx]);
      const f = bound === 0 ? (err === 0 ? 0 : Infinity) : err / bound;
      if (!(f <= worst)) worst = f;
    }
  assert(worst <= 1, `forward factor ${worst}`);
  for (let i = 0; i < a.C.length; i++)
    if (!touched[i]) assert(Object.is(got[i], a.C[i]), `C[${i}] outside the computed part changed`);
}

const gemmArgs = (c, Arr) => ({
  uplo: c.uplo, transA: c.transA, transB: c.transB, m: c.m, n: c.n, k: c.k, alpha: c.alpha,
  A: new Arr(c.A), lda: c.lda, B: new Arr(c.B), ldb: c.ldb, beta: c.beta, C: new Arr(c.C), ldc: c.ldc,
  layout: c.layout || "row-major",
});

const call = {
  sgemm: (a) => wg.sgemm(device, a.transA, a.transB, a.m, a.n, a.k, a.alpha, a.A, a.lda, a.B, a.ldb, a.beta, a.C, a.ldc, a.layout),
  sgemmtr: (a) => wg.sgemmtr(device, a.uplo, a.transA, a.transB, a.m, a.n, a.k, a.alpha, a.A, a.lda, a.B, a.ldb, a.beta, a.C, a.ldc, a.layout),
  dgemm: (a) => wg.dgemm(device, a.transA, a.transB, a.m, a.n, a.k, a.alpha, a.A, a.lda, a.B, a.ldb, a.beta, a.C, a.ldc, a.layout),
  dgemmtr: (a) => wg.dgemmtr(device, a.uplo, a.transA, a.transB, a.m, a.n, a.k, a.alpha, a.A, a.lda, a.B, a.ldb, a.beta, a.C, a.ldc, a.layout),
};

const exactEqual = (got, want, label) => {
  assertEqual(got.length, want.length, `${label}: length`);
  for (let i = 0; i < want.length; i++) assert(got[i] === want[i], `${label}: C[${i}] = ${got[i]}, want ${want[i]}`);
};

// GpuMatrix residency: the operand as wgblas's gpustorage tests build it
// (padded to outer*ld, logical shape from trans and layout).
function toGpuMatrix(X, opRows, opCols, trans, ld, layout, Arr) {
  const [rows, cols] = trans === "transpose" ? [opCols, opRows] : [opRows, opCols];
  const outer = layout === "column-major" ? cols : rows;
  const padded = new Arr(Math.max(outer * ld, X.length));
  padded.set(X);
  return wg.GpuMatrix.from(device, padded, rows, cols, ld, layout);
}

async function residentGemm(routine, a, Arr) {
  const layout = a.layout;
  const A = toGpuMatrix(a.A, a.m, a.k, a.transA, a.lda, layout, Arr);
  const B = toGpuMatrix(a.B, a.k, a.n, a.transB, a.ldb, layout, Arr);
  const C = toGpuMatrix(a.C, a.m, a.n, "no-transpose", a.ldc, layout, Arr);
  try {
    const r = await call[routine](Object.assign({}, a, { A, B, C }));
    assertEqual(Object.keys(r).length, 0, "resident call returns {}");
    const raw = new Arr(Math.max((layout === "column-major" ? a.n : a.m) * a.ldc, a.C.length));
    const dense = await C.read();
    const inner = layout === "column-major" ? a.m : a.n;
    const outer = layout === "column-major" ? a.n : a.m;
    raw.set(a.C);
    for (let o = 0; o < outer; o++) raw.set(dense.subarray(o * inner, o * inner + inner), o * a.ldc);
    return raw.subarray(0, a.C.length);
  } finally {
    A.destroy();
    B.destroy();
    C.destroy();
  }
}

// ------------------------------------------------------------- fixtures
for (const routine of ["sgemm", "sgemmtr", "dgemm", "dgemmtr"]) {
  const Arr = routine.startsWith("d") ? Float64Array : Float32Array;
  for (const file of [`${routine}.edge-cases`, `${routine}.edge-cases-column-major`]) {
    for (const c of fixture(file)) {
      test(`${routine} ${file.includes("column") ? "cm" : "rm"}: ${c.label}`, async () => {
        const a = gemmArgs(c, Arr);
        const want = refGemm(a).out;
        const got = await call[routine](a);
        if (routine.startsWith("d") && (a.alpha === 0 || a.k === 0) && a.beta === 1) {
          assert(got.C === a.C, "quick return hands back the same C");
          return;
        }
        exactEqual(got.C, want, c.label);
        exactEqual(await residentGemm(routine, a, Arr), want, `${c.label} (GpuMatrix)`);
      });
    }
  }
}

for (const routine of ["ssyrk", "dsyrk"]) {
  const Arr = routine === "dsyrk" ? Float64Array : Float32Array;
  for (const file of [`${routine}.edge-cases`, `${routine}.edge-cases-column-major`]) {
    for (const c of fixture(file)) {
      test(`${routine} ${file.includes("column") ? "cm" : "rm"}: ${c.label}`, async () => {
        const layout = c.layout || "row-major";
        const A = new Arr(c.A);
        const C = new Arr(c.C);
        const transB = c.trans === "no-transpose" ? "transpose" : "no-transpose";
        const got = await wg[routine](device, c.uplo, c.trans, c.n, c.k, c.alpha, A, c.lda, c.beta, C, c.ldc, layout);
        if (routine === "dsyrk" && (c.alpha === 0 || c.k === 0) && c.beta === 1) {
          assert(got.C === C, "quick return hands back the same C");
          return;
        }
        const want = refGemm({ uplo: c.uplo, transA: c.trans, transB, m: c.n, n: c.n, k: c.k, alpha: c.alpha, A, lda: c.lda, B: A, ldb: c.lda, beta: c.beta, C, ldc: c.ldc, layout }).out;
        exactEqual(got.C, want, c.label);
      });
    }
  }
}

const L1_EXPECT = {
  sdot: [0, 25, 0, 0, 11, 12],
  sasum: [9, 205, 0, 7, 6],
  snrm2: [5, 5, 1, 0, 5, 5, Math.fround(3e19), Math.fround(3e19)],
  isamax: [0, 0, 1, 1, 0, 3, 0, 1, 0, 1, 1],
};
const L1_KEY = { sdot: "dot", sasum: "asum", snrm2: "nrm2", isamax: "index" };
for (const routine of Object.keys(L1_EXPECT)) {
  fixture(`${routine}.edge-cases`).forEach((c, i) => {
    if (i >= L1_EXPECT[routine].length) return;
    test(`${routine}: ${c.label}`, async () => {
      const x = new Float32Array(c.x);
      const want = L1_EXPECT[routine][i];
      const host = routine === "sdot" ? await wg.sdot(device, c.n, x, c.incx, new Float32Array(c.y), c.incy)
        : await wg[routine](device, c.n, x, c.incx);
      assertEqual(host[L1_KEY[routine]], want, "host arrays");
      const gx = wg.GpuVector.from(device, x);
      const gy = routine === "sdot" ? wg.GpuVector.from(device, new Float32Array(c.y)) : null;
      try {
        const res = routine === "sdot" ? await wg.sdot(device, c.n, gx, c.incx, gy, c.incy)
          : await wg[routine](device, c.n, gx, c.incx);
        assertEqual(res[L1_KEY[routine]], want, "GpuVector");
      } finally {
        gx.destroy();
        if (gy) gy.destroy();
      }
    });
  });
}

test("level 1: n <= 0 and NaN rules", async () => {
  const x = wg.randomFloat32Array(8, -1, 1, 300);
  assertEqual((await wg.sdot(device, 0, x, 1, x, 1)).dot, 0);
  assertEqual((await wg.sasum(device, 0, x, 1)).asum, 0);
  assertEqual((await wg.snrm2(device, 0, x, 1)).nrm2, 0);
  assertEqual((await wg.isamax(device, 0, x, 1)).index, -1);
  assertEqual((await wg.isamax(device, -3, x, 1)).index, -1);
  const N = NaN;
  const I = Infinity;
  for (const [arr, want] of [[[1, N, 7, 3], 2], [[1, 2, 3, N], 2], [[N, N, N, N], 0], [[N, 5, 2, 3], 1],
    [[N, I, 2, 3], 1], [[1, I, 2, 3], 1], [[1, -I, 2, 3], 1]])
    assertEqual((await wg.isamax(device, 4, new Float32Array(arr), 1)).index, want, JSON.stringify(arr));
  const big = new Float32Array(1 << 16).fill(0.5);
  big[100] = Infinity;
  assertEqual((await wg.snrm2(device, big.length, big, 1)).nrm2, Infinity);
  big[200] = NaN;
  assert(Number.isNaN((await wg.snrm2(device, big.length, big, 1)).nrm2));
});

// level 3 on the GEMM (tests/{ssyr2k,ssymm,strmm,strsm}/): double-precision
// triple loops here; ssyr2k / ssymm / strmm within the reference's forward
// bounds, strsm by its backward residual (tests/strsm/helpers.js).
const el = (M, ld, layout, r, c) => (layout === "column-major" ? M[c * ld + r] : M[r * ld + c]);
const symEl = (A, lda, layout, uplo, r, c) =>
  (uplo === "lower" ? c <= r : c >= r) ? el(A, lda, layout, r, c) : el(A, lda, layout, c, r);
function triEl(A, lda, layout, uplo, transA, diag, r, c) {
  if (r === c) return diag === "unit" ? 1 : el(A, lda, layout, r, r);
  const lowerOp = (uplo === "lower") !== (transA === "transpose");
  if (lowerOp ? c > r : c < r) return 0;
  return transA === "transpose" ? el(A, lda, layout, c, r) : el(A, lda, layout, r, c);
}

// Storage order of operand `nm` of call `a`: its own (a.layoutA, ...), for
// GpuMatrix operands of different layouts, else the call's `layout`.
const layoutOf = (a, nm) => a["layout" + nm] || a.layout || "row-major";

// Expected output buffer and per-element bound of a level-3 call `a`.
function refLevel3(routine, a) {
  const [la, lb, lc] = [layoutOf(a, "A"), layoutOf(a, "B"), layoutOf(a, routine === "strmm" ? "B" : "C")];
  const out = Float64Array.from(routine === "strmm" ? a.B : a.C);
  const bound = new Float64Array(out.length);
  const eps = 2 ** -23;
  const rows = routine === "ssyr2k" ? a.n : a.m;
  const cols = a.n;
  for (let i = 0; i < rows; i++)
    for (let j = 0; j < cols; j++) {
      let s = 0;
      let d = 0;
      let coef;
      if (routine === "ssyr2k") {
        if (!inTri(a.uplo, i, j)) continue;
        const t = a.trans;
        for (let p = 0; p < a.k; p++) {
          const v = opElem(a.A, a.lda, la, t, i, p) * opElem(a.B, a.ldb, lb, t, j, p) +
            opElem(a.B, a.ldb, lb, t, i, p) * opElem(a.A, a.lda, la, t, j, p);
          s += v;
          d += Math.abs(opElem(a.A, a.lda, la, t, i, p) * opElem(a.B, a.ldb, lb, t, j, p)) +
            Math.abs(opElem(a.B, a.ldb, lb, t, i, p) * opElem(a.A, a.lda, la, t, j, p));
        }
        coef = a.k + 3;
      } else {
        const order = a.side === "left" ? a.m : a.n;
        for (let p = 0; p < order; p++) {
          let v;
          if (routine === "ssymm")
            v = a.side === "left" ? symEl(a.A, a.lda, la, a.uplo, i, p) * el(a.B, a.ldb, lb, p, j)
              : el(a.B, a.ldb, lb, i, p) * symEl(a.A, a.lda, la, a.uplo, p, j);
          else
            v = a.side === "left" ? triEl(a.A, a.lda, la, a.uplo, a.transA, a.diag, i, p) * el(a.B, a.ldb, lb, p, j)
              : el(a.B, a.ldb, lb, i, p) * triEl(a.A, a.lda, la, a.uplo, a.transA, a.diag, p, j);
          s += v;
          d += Math.abs(v);
        }
        coef = order + 1;
      }
      const ld = routine === "strmm" ? a.ldb : a.ldc;
      const idx = cIndex(ld, lc, i, j);
      const cin = routine === "strmm" ? 0 : a.C[idx];
      out[idx] = (a.alpha === 0 ? 0 : a.alpha * s) + (routine === "strmm" || a.beta === 0 ? 0 : a.beta * cin);
      bound[idx] = eps * (coef * Math.abs(a.alpha) * d + (routine === "strmm" ? 0 : 3 * Math.abs(a.beta) * Math.abs(cin)));
      bound[idx] += 1e-300;  // marks the element as computed
    }
  return { out, bound };
}

function checkLevel3(routine, got, a) {
  const { out, bound } = refLevel3(routine, a);
  const orig = routine === "strmm" ? a.B : a.C;
  for (let i = 0; i < out.length; i++) {
    if (bound[i] === 0) assert(Object.is(got[i], orig[i]), `${routine}: element ${i} outside the output changed`);
    else assert(Math.abs(got[i] - out[i]) <= bound[i], `${routine}: element ${i} = ${got[i]}, want ${out[i]}`);
  }
}

function trsmResidual(X, a) {
  const layout = a.layout || "row-major";
  const order = a.side === "left" ? a.m : a.n;
  let worst = 0;
  for (let i = 0; i < a.m; i++)
    for (let j = 0; j < a.n; j++) {
      let acc = 0;
      let d = 0;
      for (let k = 0; k < order; k++) {
        const [av, xv] = a.side === "left"
          ? [triEl(a.A, a.lda, layout, a.uplo, a.transA, a.diag, i, k), el(X, a.ldb, layout, k, j)]
          : [triEl(a.A, a.lda, layout, a.uplo, a.transA, a.diag, k, j), el(X, a.ldb, layout, i, k)];
        acc += av * xv;
        d += Math.abs(av * xv);
      }
      const rhs = a.alpha === 0 ? 0 : a.alpha * el(a.B, a.ldb, layout, i, j);
      const bound = 2 ** -23 * (order + 1) * d;
      const err = Math.abs(acc - rhs);
      const f = bound === 0 ? (err === 0 ? 0 : Infinity) : err / bound;
      if (!(f <= worst)) worst = f;
    }
  return worst;
}

const level3Call = {
  ssyr2k: (a) => wg.ssyr2k(device, a.uplo, a.trans, a.n, a.k, a.alpha, a.A, a.lda, a.B, a.ldb, a.beta, a.C, a.ldc, a.layout),
  ssymm: (a) => wg.ssymm(device, a.side, a.uplo, a.m, a.n, a.alpha, a.A, a.lda, a.B, a.ldb, a.beta, a.C, a.ldc, a.layout),
  strmm: (a) => wg.strmm(device, a.side, a.uplo, a.transA, a.diag, a.m, a.n, a.alpha, a.A, a.lda, a.B, a.ldb, a.layout),
  strsm: (a) => wg.strsm(device, a.side, a.uplo, a.transA, a.diag, a.m, a.n, a.alpha, a.A, a.lda, a.B, a.ldb, a.layout),
};

// GpuMatrix forms of a level-3 call's operands (shapes as wgblas's
// gpustorage tests build them) and the output read back with its ld.
async function residentLevel3(routine, a) {
  const mats = {};
  const shape = (name) => {
    if (routine === "ssyr2k") {
      if (name === "C") return [a.n, a.n, a.ldc];
      const ld = name === "A" ? a.lda : a.ldb;
      return a.trans === "no-transpose" ? [a.n, a.k, ld] : [a.k, a.n, ld];
    }
    if (name === "A") {
      const order = a.side === "left" ? a.m : a.n;
      return [order, order, a.lda];
    }
    return [a.m, a.n, name === "B" ? a.ldb : a.ldc];
  };
  const names = routine === "strmm" || routine === "strsm" ? ["A", "B"] : ["A", "B", "C"];
  const outName = routine === "strmm" || routine === "strsm" ? "B" : "C";
  try {
    for (const nm of names) {
      const [r, c, ld] = shape(nm);
      const outer = layoutOf(a, nm) === "column-major" ? c : r;
      const padded = new Float32Array(Math.max(outer * ld, a[nm].length));
      padded.set(a[nm]);
      mats[nm] = wg.GpuMatrix.from(device, padded, r, c, ld, layoutOf(a, nm));
    }
    const res = await level3Call[routine](Object.assign({}, a, mats));
    assertEqual(Object.keys(res).length, 0, "resident call returns {}");
    const [r, c, ld] = shape(outName);
    const dense = await mats[outName].read();
    const inner = layoutOf(a, outName) === "column-major" ? r : c;
    const outer = layoutOf(a, outName) === "column-major" ? c : r;
    const raw = Float32Array.from(a[outName]);
    for (let o = 0; o < outer; o++) raw.set(dense.subarray(o * inner, o * inner + inner), o * ld);
    return raw;
  } finally {
    for (const nm of Object.keys(mats)) mats[nm].destroy();
  }
}

const f32 = (c, names) => {
  const a = Object.assign({}, c);
  for (const nm of names) a[nm] = new Float32Array(c[nm]);
  a.layout = c.layout || "row-major";
  return a;
};

for (const routine of ["ssyr2k", "ssymm", "strmm", "strsm"]) {
  for (const file of [`${routine}.edge-cases`, `${routine}.edge-cases-column-major`]) {
    for (const c of fixture(file)) {
      test(`${routine} ${file.includes("column") ? "cm" : "rm"}: ${c.label}`, async () => {
        const a = f32(c, routine === "strmm" || routine === "strsm" ? ["A", "B"] : ["A", "B", "C"]);
        const key = routine === "strmm" || routine === "strsm" ? "B" : "C";
        const host = (await level3Call[routine](a))[key];
        const resident = await residentLevel3(routine, a);
        for (const got of [host, resident]) {
          if (routine === "strsm") assert(trsmResidual(got, a) <= 1, `${c.label}: residual`);
          else checkLevel3(routine, got, a);
        }
      });
    }
  }
}

test("level 3: multi-tile, mixed GpuMatrix layouts, alpha = 0, strsm many blocks", async () => {
  // ssyr2k with A row-major and B column-major GpuMatrix operands
  const n = 150;
  const k = 9;
  const A = wg.randomFloat32Array(n * k, -1, 1, 71);
  const B = wg.randomFloat32Array(n * k, -1, 1, 72);
  const C = wg.randomFloat32Array(n * n, -1, 1, 73);
  const gA = wg.GpuMatrix.from(device, A, n, k, k, "row-major");
  const gB = wg.GpuMatrix.from(device, B, n, k, n, "column-major");
  const gC = wg.GpuMatrix.from(device, C, n, n, n, "row-major");
  try {
    await wg.ssyr2k(device, "lower", "no-transpose", n, k, 1.5, gA, k, gB, n, 0.5, gC, n);
    const got = await gC.read();
    for (let i = 0; i < n; i++)
      for (let j = 0; j < n; j++) {
        if (j > i) {
          assert(Object.is(got[i * n + j], C[i * n + j]), "upper triangle untouched");
          continue;
        }
        let s = 0;
        let d = 0;
        for (let p = 0; p < k; p++) {
          const v1 = A[i * k + p] * B[p * n + j];
          const v2 = B[p * n + i] * A[j * k + p];
          s += v1 + v2;
          d += Math.abs(v1) + Math.abs(v2);
        }
        const want = 1.5 * s + 0.5 * C[i * n + j];
        assert(Math.abs(got[i * n + j] - want) <= 2 ** -23 * ((k + 3) * 1.5 * d + 1.5 * Math.abs(C[i * n + j])),
          `ssyr2k mixed layouts (${i}, ${j})`);
      }
  } finally {
    gA.destroy();
    gB.destroy();
    gC.destroy();
  }
  // ssymm / strmm multi-tile in both layouts (tests/ssymm/src/test.ssymm.js:236-297)
  for (const layout of ["row-major", "column-major"])
    for (const side of ["left", "right"]) {
      const N = 400;
      const other = 72;
      const m = side === "left" ? N : other;
      const nn = side === "left" ? other : N;
      const ld = (layout === "column-major" ? m : nn) + 4;
      const outer = layout === "column-major" ? nn : m;
      const a = { side, uplo: "upper", m, n: nn, alpha: 1.5, beta: 0.5, layout, transA: "transpose", diag: "unit",
        A: wg.randomFloat32Array(N * N, -1, 1, 91), lda: N, B: wg.randomFloat32Array(outer * ld, -1, 1, 92), ldb: ld,
        C: wg.randomFloat32Array(outer * ld, -1, 1, 93), ldc: ld };
      checkLevel3("ssymm", (await level3Call.ssymm(a)).C, a);
      checkLevel3("strmm", (await level3Call.strmm(a)).B, a);
    }
  // alpha = 0: strmm / strsm give zeros without reading NaN / Inf
  const z = { side: "left", uplo: "lower", transA: "no-transpose", diag: "non-unit", m: 7, n: 7, alpha: 0,
    A: wg.randomFloat32Array(49, -1, 1, 1), lda: 7, B: wg.randomFloat32Array(49, -1, 1, 2), ldb: 7, layout: "row-major" };
  z.A[3 * 7 + 1] = NaN;
  z.B[2 * 7 + 3] = Infinity;
  for (const r of ["strmm", "strsm"]) {
    const got = (await level3Call[r](z)).B;
    assert(got.every((v) => Object.is(v, 0)), `${r} alpha = 0 writes +0`);
  }
  // strsm across several diagonal blocks, resident, column-major with padding
  const N = 600;
  const A2 = wg.randomFloat32Array(N * N, -1 / N, 1 / N, 121);
  for (let i = 0; i < N; i++) A2[i * N + i] = 2;
  const s = { side: "right", uplo: "lower", transA: "transpose", diag: "non-unit", m: 200, n: N, alpha: 1.5,
    A: A2, lda: N, B: wg.randomFloat32Array(N * 204, -1, 1, 122), ldb: 204, layout: "column-major" };
  assert(trsmResidual(await residentLevel3("strsm", s), s) <= 1, "strsm 600 resident residual");
});

// sgemv (tests/sgemv/): the fixtures exactly (as the reference's
// assert.deepEqual against stdlib), host arrays and GpuMatrix / GpuVector
function refGemv(c) {
  const layout = c.layout || "row-major";
  const at = (r, k) => (layout === "column-major" ? c.A[k * c.lda + r] : c.A[r * c.lda + k]);
  const noT = c.trans === "no-transpose";
  const yLen = noT ? c.m : c.n;
  const out = Float64Array.from(c.y);
  for (let i = 0; i < yLen; i++) {
    let s = 0;
    for (let p = 0; p < (noT ? c.n : c.m); p++) s += (noT ? at(i, p) : at(p, i)) * c.x[p * c.incx];
    out[i * c.incy] = (c.alpha === 0 ? 0 : c.alpha * s) + (c.beta === 0 ? 0 : c.beta * c.y[i * c.incy]);
  }
  return out;
}
for (const file of ["sgemv.edge-cases", "sgemv.edge-cases-column-major"]) {
  for (const c of fixture(file)) {
    test(`sgemv ${file.includes("column") ? "cm" : "rm"}: ${c.label}`, async () => {
      const layout = c.layout || "row-major";
      const A = new Float32Array(c.A);
      const x = new Float32Array(c.x);
      const y = new Float32Array(c.y);
      const want = refGemv(Object.assign({}, c, { layout }));
      const got = await wg.sgemv(device, c.trans, c.m, c.n, c.alpha, A, c.lda, x, c.incx, c.beta, y, c.incy, layout);
      exactEqual(got.y, want, c.label);
      const outer = layout === "column-major" ? c.n : c.m;
      const padded = new Float32Array(Math.max(outer * c.lda, A.length));
      padded.set(A);
      const gA = wg.GpuMatrix.from(device, padded, c.m, c.n, c.lda, layout);
      const gx = wg.GpuVector.from(device, x);
      const gy = wg.GpuVector.from(device, y);
      try {
        const r = await wg.sgemv(device, c.trans, c.m, c.n, c.alpha, gA, c.lda, gx, c.incx, c.beta, gy, c.incy, layout);
        assertEqual(Object.keys(r).length, 0, "resident call returns {}");
        exactEqual(await gy.read(), want, `${c.label} (GpuVector)`);
      } finally {
        gA.destroy();
        gx.destroy();
        gy.destroy();
      }
    });
  }
}

test("sgemv: 600 x 300 split paths, zero dimension", async () => {
  for (const layout of ["row-major", "column-major"])
    for (const trans of ["no-transpose", "transpose"]) {
      const [m, n] = layout === "row-major" ? [600, 300] : [300, 600];
      const noT = trans === "no-transpose";
      const c = { layout, trans, m, n, alpha: 1.5, beta: 0.75, incx: 3, incy: 2,
        A: wg.randomFloat32Array(m * n, -1, 1, 21), lda: layout === "row-major" ? n : m };
      c.x = wg.randomFloat32Array(((noT ? n : m) - 1) * 3 + 1, -1, 1, 22);
      c.y = wg.randomFloat32Array(((noT ? m : n) - 1) * 2 + 1, -1, 1, 23);
      const got = (await wg.sgemv(device, trans, m, n, c.alpha, c.A, c.lda, c.x, c.incx, c.beta, c.y, c.incy, layout)).y;
      const want = refGemv(c);
      const terms = noT ? n : m;
      for (let i = 0; i < want.length; i++) {
        if (i % 2) {
          assert(Object.is(got[i], c.y[i]), "incy gap untouched");
          continue;
        }
        assert(Math.abs(got[i] - want[i]) <= 2 ** -23 * (terms + 1) * 1.5 * terms + 1e-6, `${layout} ${trans} y[${i}]`);
      }
    }
  const y = wg.randomFloat32Array(4, -1, 1, 9001);
  const r = await wg.sgemv(device, "no-transpose", 4, 0, 1.5, new Float32Array(0), 1, new Float32Array(0), 1, 0.5, y, 1);
  exactEqual(r.y, y, "n = 0 leaves y");
});

// fp64 level 1 (tests/{ddot,dasum,dnrm2,idamax}/): the reference's bounds
// around float64 sums (ddot n 2^-48 sum|xy|, dasum 64 ULP by a relative
// 64 * 2^-52, dnrm2 10 * 2^-48 relative), idamax exact
const IDAMAX_EXPECT = [0, 0, 1, 1, 0, 3, 0, 1, 0, 1, 1, 1];
const D_KEY = { ddot: "dot", dasum: "asum", dnrm2: "nrm2", idamax: "index" };
function refD(routine, c) {
  let s = 0;
  let a = 0;
  for (let i = 0; i < c.n; i++) {
    const xv = c.x[i * c.incx];
    if (routine === "ddot") {
      s += xv * c.y[i * c.incy];
      a += Math.abs(xv * c.y[i * c.incy]);
    } else if (routine === "dasum") s += Math.abs(xv);
    else s = Math.hypot(s, xv);
  }
  if (routine === "ddot") return { want: s, tol: c.n * 2 ** -48 * a };
  if (routine === "dasum") return { want: s, tol: 64 * 2 ** -52 * s };
  return { want: s, tol: 10 * 2 ** -48 * s };
}
for (const routine of Object.keys(D_KEY)) {
  fixture(`${routine}.edge-cases`).forEach((c, i) => {
    test(`${routine}: ${c.label}`, async () => {
      const x = new Float64Array(c.x);
      const args = routine === "ddot" ? [c.n, x, c.incx, new Float64Array(c.y), c.incy] : [c.n, x, c.incx];
      const check = (got, how) => {
        if (routine === "idamax") return assertEqual(got, IDAMAX_EXPECT[i], how);
        const { want, tol } = refD(routine, c);
        assert(Math.abs(got - want) <= tol, `${how}: ${got} vs ${want}`);
      };
      check((await wg[routine](device, ...args))[D_KEY[routine]], "host arrays");
      const gx = wg.GpuVector.from(device, x);
      const gy = routine === "ddot" ? wg.GpuVector.from(device, new Float64Array(c.y)) : null;
      try {
        const res = routine === "ddot" ? await wg.ddot(device, c.n, gx, c.incx, gy, c.incy)
          : await wg[routine](device, c.n, gx, c.incx);
        check(res[D_KEY[routine]], "GpuVector");
      } finally {
        gx.destroy();
        if (gy) gy.destroy();
      }
    });
  });
}

test("fp64 level 1: n <= 0, NaN rules, f64 range, long strided vectors", async () => {
  const x = wg.randomFloat64Array(8, -1, 1, 300);
  assertEqual((await wg.ddot(device, 0, x, 1, x, 1)).dot, 0);
  assertEqual((await wg.dasum(device, 0, x, 1)).asum, 0);
  assertEqual((await wg.dnrm2(device, 0, x, 1)).nrm2, 0);
  assertEqual((await wg.idamax(device, 0, x, 1)).index, -1);
  const N = NaN;
  const I = Infinity;
  for (const [arr, want] of [[[1, N, 7, 3], 2], [[N, N, N, N], 0], [[N, I, 2, 3], 1], [[1, -I, 2, 3], 1],
    [[1e300, 1e301, 5, 1], 1]])
    assertEqual((await wg.idamax(device, 4, new Float64Array(arr), 1)).index, want, JSON.stringify(arr));
  assertEqual((await wg.dnrm2(device, 2, new Float64Array([3e300, 4e300]), 1)).nrm2, 5e300);
  const n = 100003;
  const inc = 3;
  const v = wg.randomFloat64Array((n - 1) * inc + 1, -1, 1, 17);
  const w = wg.randomFloat64Array((n - 1) * inc + 1, -1, 1, 18);
  const c = { n, x: v, y: w, incx: inc, incy: inc };
  const gv = wg.GpuVector.from(device, v);
  const gw = wg.GpuVector.from(device, w);
  try {
    for (const routine of ["ddot", "dasum", "dnrm2"]) {
      const res = routine === "ddot" ? await wg.ddot(device, n, gv, inc, gw, inc) : await wg[routine](device, n, gv, inc);
      const { want, tol } = refD(routine, c);
      // long sums: the float64 reference itself carries n 2^-53 relative error
      const slack = routine === "ddot" ? 0 : n * 2 ** -53 * want;
      assert(Math.abs(res[D_KEY[routine]] - want) <= tol + slack, `${routine}: ${res[D_KEY[routine]]} vs ${want}`);
    }
    let best = 0;
    for (let i = 1; i < n; i++) if (Math.abs(v[i * inc]) > Math.abs(v[best * inc])) best = i;
    assertEqual((await wg.idamax(device, n, gv, inc)).index, best);
  } finally {
    gv.destroy();
    gw.destroy();
  }
});

// ------------------------------------------------------------ regressions
for (const layout of ["row-major", "column-major"])
  for (const transA of ["no-transpose", "transpose"])
    for (const transB of ["no-transpose", "transpose"]) {
      test(`sgemm ${layout} ${transA}/${transB}: 398x390x13 ld rounded to 4 (host and GpuMatrix)`, async () => {
        const M = 398;
        const N = 390;
        const K = 13;
        const cm = layout === "column-major";
        const up4 = (v) => Math.ceil(v / 4) * 4;
        const [aR, aC] = transA === "no-transpose" ? [M, K] : [K, M];
        const [bR, bC] = transB === "no-transpose" ? [K, N] : [N, K];
        const lda = up4(cm ? aR : aC);
        const ldb = up4(cm ? bR : bC);
        const a = { transA, transB, m: M, n: N, k: K, alpha: 1.5, beta: 0.5, lda, ldb, ldc: cm ? M : N, layout,
          A: wg.randomFloat32Array((cm ? aC : aR) * lda, -1, 1, 111), B: wg.randomFloat32Array((cm ? bC : bR) * ldb, -1, 1, 112),
          C: wg.randomFloat32Array(M * N, -1, 1, 113) };
        checkGemm((await call.sgemm(a)).C, a, false);
        checkGemm(await residentGemm("sgemm", a, Float32Array), a, false);
      });
    }

for (const layout of ["row-major", "column-major"])
  for (const [M, N] of [[150, 70], [70, 150]])
    for (const uplo of ["lower", "upper"]) {
      test(`sgemmtr ${layout} ${M}x${N} ${uplo}: other triangle untouched`, async () => {
        const cm = layout === "column-major";
        const K = 9;
        const a = { uplo, transA: "transpose", transB: "no-transpose", m: M, n: N, k: K, alpha: 1.5, beta: 0.5,
          A: wg.randomFloat32Array(K * M, -1, 1, 51), lda: cm ? K : M, B: wg.randomFloat32Array(K * N, -1, 1, 52),
          ldb: cm ? K : N, C: wg.randomFloat32Array(M * N, -1, 1, 53), ldc: cm ? M : N, layout };
        checkGemm((await call.sgemmtr(a)).C, a, false);
      });
    }

for (const layout of ["row-major", "column-major"])
  for (const uplo of ["lower", "upper"])
    for (const trans of ["no-transpose", "transpose"]) {
      test(`ssyrk ${layout} ${uplo} ${trans}: 301x64, GpuMatrix chained x3`, async () => {
        const n = 301;
        const k = 64;
        const cm = layout === "column-major";
        const [aR, aC] = trans === "no-transpose" ? [n, k] : [k, n];
        const lda = cm ? aR : aC;
        const A = wg.randomFloat32Array(aR * aC, -1, 1, 61);
        let C = wg.randomFloat32Array(n * n, -1, 1, 62);
        const gA = wg.GpuMatrix.from(device, A, aR, aC, lda, layout);
        const gC = wg.GpuMatrix.from(device, C, n, n, n, layout);
        const transB = trans === "no-transpose" ? "transpose" : "no-transpose";
        try {
          for (let it = 0; it < 3; it++) {
            const a = { uplo, transA: trans, transB, m: n, n, k, alpha: 1, beta: 0.25, A, lda, B: A, ldb: lda, C, ldc: n, layout };
            const r = await wg.ssyrk(device, uplo, trans, n, k, 1, gA, lda, 0.25, gC, n);
            assertEqual(Object.keys(r).length, 0, "resident call returns {}");
            const got = await gC.read();
            checkGemm(got, a, false);
            C = got;
          }
        } finally {
          gA.destroy();
          gC.destroy();
        }
      });
    }

test("sgemm k = 0 is beta*C bit-exact; alpha = 0 reads neither A nor B", async () => {
  const C = wg.randomFloat32Array(16, -5, 5, 300);
  const r = await wg.sgemm(device, "no-transpose", "transpose", 4, 4, 0, 1.5, new Float32Array(3), 1, new Float32Array(3), 1, 0.5, C, 4);
  for (let i = 0; i < 16; i++) assert(Object.is(r.C[i], Math.fround(0.5 * C[i])), `element ${i}`);
  for (const beta of [0, 0.5]) {
    const n = 400;
    const A = wg.randomFloat32Array(n * n, -1, 1, 1);
    const B = wg.randomFloat32Array(n * n, -1, 1, 2);
    const C2 = wg.randomFloat32Array(n * n, -1, 1, 3);
    A[n + 2] = NaN;
    B[2 * n + 3] = Infinity;
    if (beta === 0) C2[4 * n + 4] = NaN;
    const g = await wg.sgemm(device, "no-transpose", "no-transpose", n, n, n, 0, A, n, B, n, beta, C2, n);
    for (let i = 0; i < n * n; i++) assert(Object.is(g.C[i], beta === 0 ? 0 : Math.fround(beta * C2[i])), `alpha=0 C[${i}]`);
  }
});

test("dgemm: random 150x133x77 within the double-double bound, all layouts/trans", async () => {
  for (const layout of ["row-major", "column-major"])
    for (const transA of ["no-transpose", "transpose"])
      for (const transB of ["no-transpose", "transpose"]) {
        const M = 150;
        const N = 133;
        const K = 77;
        const cm = layout === "column-major";
        const [aR, aC] = transA === "no-transpose" ? [M, K] : [K, M];
        const [bR, bC] = transB === "no-transpose" ? [K, N] : [N, K];
        const a = { transA, transB, m: M, n: N, k: K, alpha: 1.25, beta: -0.5, layout,
          A: wg.randomFloat64Array(aR * aC, -1, 1, 3), lda: cm ? aR : aC,
          B: wg.randomFloat64Array(bR * bC, -1, 1, 4), ldb: cm ? bR : bC,
          C: wg.randomFloat64Array(M * N, -1, 1, 5), ldc: cm ? M : N };
        checkGemm((await call.dgemm(a)).C, a, true);
      }
});

test("dgemmtr / dsyrk: random within the double-double bound, resident and host", async () => {
  for (const layout of ["row-major", "column-major"])
    for (const uplo of ["lower", "upper"]) {
      const cm = layout === "column-major";
      const M = 140;
      const N = 95;
      const K = 70;
      const a = { uplo, transA: "no-transpose", transB: "transpose", m: M, n: N, k: K, alpha: 1.25, beta: -0.5, layout,
        A: wg.randomFloat64Array(M * K, -1, 1, 7), lda: cm ? M : K,
        B: wg.randomFloat64Array(N * K, -1, 1, 8), ldb: cm ? N : K,
        C: wg.randomFloat64Array(M * N, -1, 1, 9), ldc: cm ? M : N };
      checkGemm((await call.dgemmtr(a)).C, a, true);
      checkGemm(await residentGemm("dgemmtr", a, Float64Array), a, true);
      for (const trans of ["no-transpose", "transpose"]) {
        const n = 130;
        const k = 40;
        const [aR, aC] = trans === "no-transpose" ? [n, k] : [k, n];
        const lda = cm ? aR : aC;
        const A = wg.randomFloat64Array(aR * aC, -1, 1, 10);
        const C = wg.randomFloat64Array(n * n, -1, 1, 11);
        const transB = trans === "no-transpose" ? "transpose" : "no-transpose";
        const s = { uplo, transA: trans, transB, m: n, n, k, alpha: 1, beta: 0.25, A, lda, B: A, ldb: lda, C, ldc: n, layout };
        checkGemm((await wg.dsyrk(device, uplo, trans, n, k, 1, A, lda, 0.25, C, n, layout)).C, s, true);
        const gA = wg.GpuMatrix.from(device, A, aR, aC, lda, layout);
        const gC = wg.GpuMatrix.from(device, C, n, n, n, layout);
        try {
          const r = await wg.dsyrk(device, uplo, trans, n, k, 1, gA, lda, 0.25, gC, n);
          assertEqual(Object.keys(r).length, 0, "resident call returns {}");
          checkGemm(await gC.read(), s, true);
        } finally {
          gA.destroy();
          gC.destroy();
        }
      }
    }
});

// ssymm with B and C of different storage orders, and ssyr2k with A and B of
// different storage orders (GpuMatrix operands carry their own layout;
// wgblas accepts both: src/ssymm/ssymm.mjs:85-87, 149-163,
// src/ssyr2k/ssyr2k.mjs:149-205).
for (const [lB, lC] of [["row-major", "column-major"], ["column-major", "row-major"]])
  for (const side of ["left", "right"])
    test(`ssymm GpuMatrix B ${lB}, C ${lC}, side ${side}`, async () => {
      const [m, n] = side === "left" ? [70, 45] : [45, 70];
      const order = side === "left" ? m : n;
      const ldb = (lB === "column-major" ? m : n) + 2;
      const ldc = (lC === "column-major" ? m : n) + 1;
      const a = { side, uplo: "lower", m, n, alpha: 1.25, beta: 0.5, layoutA: "column-major", layoutB: lB, layoutC: lC,
        A: wg.randomFloat32Array(order * order, -1, 1, 71), lda: order,
        B: wg.randomFloat32Array((lB === "column-major" ? n : m) * ldb, -1, 1, 72), ldb,
        C: wg.randomFloat32Array((lC === "column-major" ? n : m) * ldc, -1, 1, 73), ldc };
      checkLevel3("ssymm", await residentLevel3("ssymm", a), a);
    });

for (const [lA, lB] of [["row-major", "column-major"], ["column-major", "row-major"]])
  for (const trans of ["no-transpose", "transpose"])
    test(`ssyr2k GpuMatrix A ${lA}, B ${lB}, ${trans}`, async () => {
      const n = 90;
      const k = 33;
      const [r, c] = trans === "no-transpose" ? [n, k] : [k, n];
      const lda = (lA === "column-major" ? r : c) + 1;
      const ldb = (lB === "column-major" ? r : c) + 3;
      const a = { uplo: "upper", trans, n, k, alpha: 0.75, beta: -0.5, layoutA: lA, layoutB: lB, layoutC: "row-major",
        A: wg.randomFloat32Array((lA === "column-major" ? c : r) * lda, -1, 1, 74), lda,
        B: wg.randomFloat32Array((lB === "column-major" ? c : r) * ldb, -1, 1, 75), ldb,
        C: wg.randomFloat32Array(n * n, -1, 1, 76), ldc: n };
      checkLevel3("ssyr2k", await residentLevel3("ssyr2k", a), a);
    });

// fp32 routines given a Float64Array-backed resident operand compute on its
// float32 rounding, as wgblas's fp32 routines compute on the `_buf` (float32
// high half) of such an operand (src/util/f64.mjs:33-63); an output then
// reads back as the float32 result plus its old low half. Every operand
// starts at 1 + 2^-30 (high half 1, low half 2^-30), so each call must equal
// the all-Float32Array call on ones, plus 2^-30 in an f64-backed output.
test("fp32 routines read Float64Array-backed resident operands as float32", async () => {
  const v = 1 + 2 ** -30;
  const M = (dt) => wg.GpuMatrix.from(device, new dt(64).fill(dt === Float64Array ? v : 1), 8, 8, 8, "column-major");
  const V = (dt) => wg.GpuVector.from(device, new dt(8).fill(dt === Float64Array ? v : 1));
  const N = "no-transpose";
  const cases = [
    ["sgemm", ["A", "B", "C"], "C", (o) => wg.sgemm(device, N, N, 8, 8, 8, 1, o.A, 8, o.B, 8, 0.5, o.C, 8)],
    ["sgemmtr", ["A", "B", "C"], "C", (o) => wg.sgemmtr(device, "lower", N, N, 8, 8, 8, 1, o.A, 8, o.B, 8, 0.5, o.C, 8)],
    ["ssyrk", ["A", "C"], "C", (o) => wg.ssyrk(device, "lower", N, 8, 8, 1, o.A, 8, 0.5, o.C, 8)],
    ["ssyr2k", ["A", "B", "C"], "C", (o) => wg.ssyr2k(device, "lower", N, 8, 8, 1, o.A, 8, o.B, 8, 0.5, o.C, 8)],
    ["ssymm", ["A", "B", "C"], "C", (o) => wg.ssymm(device, "left", "lower", 8, 8, 1, o.A, 8, o.B, 8, 0.5, o.C, 8)],
    ["strmm", ["A", "B"], "B", (o) => wg.strmm(device, "left", "lower", N, "non-unit", 8, 8, 1, o.A, 8, o.B, 8)],
    ["strsm", ["A", "B"], "B", (o) => wg.strsm(device, "left", "lower", N, "non-unit", 8, 8, 1, o.A, 8, o.B, 8)],
    ["sgemv", ["A", "x", "y"], "y", (o) => wg.sgemv(device, N, 8, 8, 1, o.A, 8, o.x, 1, 0.5, o.y, 1)],
    ["sdot", ["x", "y"], null, (o) => wg.sdot(device, 8, o.x, 1, o.y, 1)],
    ["sasum", ["x"], null, (o) => wg.sasum(device, 8, o.x, 1)],
    ["snrm2", ["x"], null, (o) => wg.snrm2(device, 8, o.x, 1)],
    ["isamax", ["x"], null, (o) => wg.isamax(device, 8, o.x, 1)],
  ];
  const runWith = async (names, out, fn, f64name) => {
    const o = {};
    for (const nm of names) {
      const dt = nm === f64name ? Float64Array : Float32Array;
      o[nm] = nm === "x" || nm === "y" ? V(dt) : M(dt);
    }
    try {
      const r = await fn(o);
      return out === null ? Object.values(r)[0] : Array.from(await o[out].read());
    } finally {
      for (const nm of names) o[nm].destroy();
    }
  };
  for (const [routine, names, out, fn] of cases) {
    const base = await runWith(names, out, fn, null);
    for (const f64name of names) {
      const got = await runWith(names, out, fn, f64name);
      if (out === null) {
        assertEqual(got, base, `${routine} with ${f64name} f64-backed`);
        continue;
      }
      const lo = f64name === out ? 2 ** -30 : 0;
      for (let i = 0; i < base.length; i++)
        assertEqual(got[i], base[i] + lo, `${routine} with ${f64name} f64-backed, element ${i}`);
    }
  }
});

test("GpuMatrix.read strips lda padding; GpuVector round trip", async () => {
  const data = new Float32Array([1, 2, 99, 3, 4, 99]);
  const g = wg.GpuMatrix.from(device, data, 2, 2, 3);
  exactEqual(await g.read(), new Float32Array([1, 2, 3, 4]), "row-major read");
  g.destroy();
  const v = wg.GpuVector.from(device, new Float64Array([Math.PI, -0, 1e300]));
  const back = await v.read();
  assert(back instanceof Float64Array && back[0] === Math.PI && Object.is(back[1], -0) && back[2] === 1e300);
  v.destroy();
});
