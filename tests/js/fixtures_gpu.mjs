// Random fixtures through the JavaScript API on the GPU, in the shape of
// wgblas's property-based runner (tests/helpers/fixtures.js runFixtures and
// buildArb, used by tests/<routine>/src/test.<routine>.js "<routine> fixtures"
// and gpustorage.<routine>.js): NUM_RUNS argument sets per routine drawn from
// the reference's own parameter specs (tests/golden/validation_params, its
// tests/validation/params): the string parameters from their value lists,
// scalars and array elements from their ranges, each leading dimension at its
// minimum plus 0 .. (ld.max - ld.min), arrays of exactly the length their
// shape and stride need, m / n / k capped at 1 .. 20 for the GEMM family as
// the reference's fixtureSpecs do, and nonzero values below 1e-3 in
// magnitude drawn again (floatArb's filter). Each result is held to the
// reference's metric and threshold against a float64 result computed here:
// the forward-error factor <= 1 for sgemm / sgemmtr / ssyrk
// (tests/sgemm/helpers.js: eps 2^-23, (k + 1)), dgemm (tests/dgemm/helpers.js:
// eps 2^-48, (k + 2), 3 |beta| |C|) and sdot (tests/sdot/helpers.js:
// n eps sum |x y|), 50 ULP for sasum and snrm2, the exact index for isamax.
// The same runs are made again with GpuMatrix / GpuVector operands. Elements
// a call must not write (outside the triangle, ld padding) are bit-checked.
// A seeded mulberry32 stream stands in for fast-check (not installed), so the
// runs are the same on every execution. Registered by validation.mjs --gpu.
import { readFileSync } from "fs";
import { fileURLToPath } from "url";
import { dirname, join } from "path";
import { test, assert } from "./harness.mjs";

const here = dirname(fileURLToPath(import.meta.url));
const spec = (name) =>
  JSON.parse(readFileSync(join(here, "..", "golden", "validation_params", `${name}.json`), "utf8"));

const NUM_RUNS = 100;

// mulberry32 (Tommy Ettinger's published 32-bit generator): uniform [0, 1).
function mulberry32(seed) {
  let a = seed >>> 0;
  return () => {
    a = (a + 0x6d2b79f5) >>> 0;
    let t = a;
    t = Math.imul(t ^ (t >>> 15), t | 1);
    t ^= t + Math.imul(t ^ (t >>> 7), t | 61);
    return ((t ^ (t >>> 14)) >>> 0) / 4294967296;
  };
}

class Gen {
  constructor(seed) {
    this.r = mulberry32(seed);
  }
  int(min, max) {
    return min + Math.floor(this.r() * (max - min + 1));
  }
  pick(values) {
    return values[this.int(0, values.length - 1)];
  }
  // f32 (or f64) value in [min, max], 0 or at least 1e-3 in magnitude
  num(min, max, f64 = false) {
    for (;;) {
      const x = min + (max - min) * this.r();
      const v = f64 ? x : Math.fround(x);
      if (v === 0 || Math.abs(v) >= 1e-3) return v;
    }
  }
  array(len, range, Arr) {
    const out = new Arr(len);
    for (let i = 0; i < len; i++) out[i] = this.num(range.elementMin, range.elementMax, Arr === Float64Array);
    return out;
  }
}

const S = {
  trans: spec("trans").values,
  layout: spec("layout").values,
  uplo: spec("uplo").values,
  n: spec("n").range,
  incx: spec("incx").range,
  incy: spec("incy").range,
  x: spec("x").range,
  y: spec("y").range,
  A: spec("A").range,
  B: spec("B").range,
  C: spec("C").range,
  alpha: spec("alpha").range,
  beta: spec("beta").range,
  ldPad: spec("ld").range.max - spec("ld").range.min,
};
const GEMM_DIM = { min: 1, max: 20 };

// ---------------------------------------------------------------- metrics
const f32bits = new Uint32Array(1);
const f32view = new Float32Array(f32bits.buffer);
function ulpDiff(a, b) {
  if (Math.abs(a) === 0 && Math.abs(b) === 0) return 0;
  f32view[0] = a;
  const ua = f32bits[0];
  f32view[0] = b;
  const ub = f32bits[0];
  return Math.abs(ua - ub);
}

// A stored matrix: element (r, c) of the rows x cols array in `layout`.
const at = (M, ld, layout, r, c) => (layout === "column-major" ? M[c * ld + r] : M[r * ld + c]);
const idx = (ld, layout, r, c) => (layout === "column-major" ? c * ld + r : r * ld + c);
// Minimal length of a rows x cols array with leading dimension ld.
const minLen = (rows, cols, ld, layout) =>
  layout === "column-major" ? (cols - 1) * ld + rows : (rows - 1) * ld + cols;
const ldFloor = (rows, cols, layout) => (layout === "column-major" ? rows : cols);

// One GEMM-family argument set: op(A) m x k, op(B) k x n, C m x n.
function gemmArgs(g, routine, Arr) {
  const f64 = Arr === Float64Array;
  const a = { routine, layout: g.pick(S.layout), m: g.int(GEMM_DIM.min, GEMM_DIM.max),
              n: g.int(GEMM_DIM.min, GEMM_DIM.max), k: g.int(GEMM_DIM.min, GEMM_DIM.max),
              alpha: g.num(S.alpha.min, S.alpha.max, f64), beta: g.num(S.beta.min, S.beta.max, f64) };
  if (routine === "ssyrk") {
    a.uplo = g.pick(S.uplo);
    a.trans = g.pick(S.trans);
    a.m = a.n;
    a.transA = a.trans;
    a.transB = a.trans === "transpose" ? "no-transpose" : "transpose";
  } else {
    a.transA = g.pick(S.trans);
    a.transB = g.pick(S.trans);
    if (routine === "sgemmtr") a.uplo = g.pick(S.uplo);
  }
  // stored shapes
  a.aRows = a.transA === "transpose" ? a.k : a.m;
  a.aCols = a.transA === "transpose" ? a.m : a.k;
  a.lda = ldFloor(a.aRows, a.aCols, a.layout) + g.int(0, S.ldPad);
  a.A = g.array(minLen(a.aRows, a.aCols, a.lda, a.layout), S.A, Arr);
  if (routine === "ssyrk") {
    // op(B) = op(A)^T: the same stored array
    a.bRows = a.aRows;
    a.bCols = a.aCols;
    a.ldb = a.lda;
    a.B = a.A;
  } else {
    a.bRows = a.transB === "transpose" ? a.n : a.k;
    a.bCols = a.transB === "transpose" ? a.k : a.n;
    a.ldb = ldFloor(a.bRows, a.bCols, a.layout) + g.int(0, S.ldPad);
    a.B = g.array(minLen(a.bRows, a.bCols, a.ldb, a.layout), S.B, Arr);
  }
  a.ldc = ldFloor(a.m, a.n, a.layout) + g.int(0, S.ldPad);
  a.C = g.array(minLen(a.m, a.n, a.ldc, a.layout), S.C, Arr);
  return a;
}

const opAt = (M, ld, layout, trans, r, c) => (trans === "transpose" ? at(M, ld, layout, c, r) : at(M, ld, layout, r, c));
const inTri = (uplo, i, j) => !uplo || (uplo === "lower" ? i >= j : i <= j);

// Largest forward-error factor of C over the computed part, and whether
// every other element kept its bits.
function gemmFactor(gotC, a, f64) {
  const eps = f64 ? 2 ** -48 : 2 ** -23;
  let worst = 0;
  const written = new Uint8Array(a.C.length);
  for (let i = 0; i < a.m; i++)
    for (let j = 0; j < a.n; j++) {
      if (!inTri(a.uplo, i, j)) continue;
      let s = 0;
      let sa = 0;
      for (let p = 0; p < a.k; p++) {
        const prod = opAt(a.A, a.lda, a.layout, a.transA, i, p) * opAt(a.B, a.ldb, a.layout, a.transB, p, j);
        s += prod;
        sa += Math.abs(prod);
      }
      const q = idx(a.ldc, a.layout, i, j);
      written[q] = 1;
      const ref = a.alpha * s + a.beta * a.C[q];
      const bound = eps * ((a.k + (f64 ? 2 : 1)) * Math.abs(a.alpha) * sa +
                           (f64 ? 3 : 1) * Math.abs(a.beta) * Math.abs(a.C[q]));
      const err = Math.abs(gotC[q] - ref);
      const f = bound === 0 ? (err === 0 ? 0 : Infinity) : err / bound;
      if (!(f <= worst)) worst = f;
    }
  for (let q = 0; q < a.C.length; q++)
    if (!written[q] && !Object.is(gotC[q], a.C[q])) return { worst, untouched: false };
  return { worst, untouched: true };
}

async function callGemm(wg, device, a, A, B, C) {
  if (a.routine === "ssyrk")
    return wg.ssyrk(device, a.uplo, a.trans, a.n, a.k, a.alpha, A, a.lda, a.beta, C, a.ldc, a.layout);
  if (a.routine === "sgemmtr")
    return wg.sgemmtr(device, a.uplo, a.transA, a.transB, a.m, a.n, a.k, a.alpha, A, a.lda, B, a.ldb, a.beta, C,
                      a.ldc, a.layout);
  return wg[a.routine](device, a.transA, a.transB, a.m, a.n, a.k, a.alpha, A, a.lda, B, a.ldb, a.beta, C, a.ldc,
                       a.layout);
}

// A stored array as a GpuMatrix (padded to outer * ld, as GpuMatrix.from
// requires), and C read back into a copy of the stored array.
function toGpu(wg, device, X, rows, cols, ld, layout, Arr) {
  const outer = layout === "column-major" ? cols : rows;
  const padded = new Arr(outer * ld);
  padded.set(X);
  return wg.GpuMatrix.from(device, padded, rows, cols, ld, layout);
}

async function gemmRun(wg, device, a, Arr, resident) {
  if (!resident) return (await callGemm(wg, device, a, a.A, a.B, a.C)).C;
  const A = toGpu(wg, device, a.A, a.aRows, a.aCols, a.lda, a.layout, Arr);
  const B = a.routine === "ssyrk" ? A : toGpu(wg, device, a.B, a.bRows, a.bCols, a.ldb, a.layout, Arr);
  const C = toGpu(wg, device, a.C, a.m, a.n, a.ldc, a.layout, Arr);
  try {
    await callGemm(wg, device, a, A, B, C);
    const dense = await C.read();
    const out = Arr.from(a.C);
    const inner = a.layout === "column-major" ? a.m : a.n;
    const outer = a.layout === "column-major" ? a.n : a.m;
    for (let o = 0; o < outer; o++)
      for (let e = 0; e < inner; e++) out[o * a.ldc + e] = dense[o * inner + e];
    return out;
  } finally {
    A.destroy();
    if (B !== A) B.destroy();
    C.destroy();
  }
}

// ------------------------------------------------------------- level 1
function vecArgs(g, two) {
  const a = { n: g.int(S.n.min, S.n.max), incx: g.int(S.incx.min, S.incx.max) };
  a.x = g.array((a.n - 1) * a.incx + 1, S.x, Float32Array);
  if (two) {
    a.incy = g.int(S.incy.min, S.incy.max);
    a.y = g.array((a.n - 1) * a.incy + 1, S.y, Float32Array);
  }
  return a;
}

const L1 = {
  sdot: {
    two: true,
    call: (wg, d, a, x, y) => wg.sdot(d, a.n, x, a.incx, y, a.incy).then((r) => r.dot),
    metric: (got, a) => {
      let s = 0;
      let sa = 0;
      for (let i = 0; i < a.n; i++) {
        const p = a.x[i * a.incx] * a.y[i * a.incy];
        s += p;
        sa += Math.abs(p);
      }
      const bound = a.n * 2 ** -23 * sa;
      return bound === 0 ? (got === s ? 0 : Infinity) : Math.abs(got - s) / bound;
    },
    threshold: 1,
  },
  sasum: {
    call: (wg, d, a, x) => wg.sasum(d, a.n, x, a.incx).then((r) => r.asum),
    metric: (got, a) => {
      let s = 0;
      for (let i = 0; i < a.n; i++) s += Math.abs(a.x[i * a.incx]);
      return ulpDiff(got, Math.fround(s));
    },
    threshold: 50,
  },
  snrm2: {
    call: (wg, d, a, x) => wg.snrm2(d, a.n, x, a.incx).then((r) => r.nrm2),
    metric: (got, a) => {
      let s = 0;
      for (let i = 0; i < a.n; i++) s += a.x[i * a.incx] * a.x[i * a.incx];
      return ulpDiff(got, Math.fround(Math.sqrt(s)));
    },
    threshold: 50,
  },
  isamax: {
    call: (wg, d, a, x) => wg.isamax(d, a.n, x, a.incx).then((r) => r.index),
    metric: (got, a) => {
      let best = 0;
      for (let i = 1; i < a.n; i++) if (Math.abs(a.x[i * a.incx]) > Math.abs(a.x[best * a.incx])) best = i;
      return got === best ? 0 : 1;
    },
    threshold: 0,
  },
};

export function registerFixtureTests(wg, device) {
  const seeds = { sgemm: 101, sgemmtr: 102, ssyrk: 103, dgemm: 104, sdot: 105, sasum: 106, snrm2: 107, isamax: 108 };
  for (const routine of ["sgemm", "sgemmtr", "ssyrk", "dgemm"]) {
    const Arr = routine === "dgemm" ? Float64Array : Float32Array;
    for (const resident of [false, true]) {
      test(`fixtures: ${routine}, ${NUM_RUNS} random runs${resident ? " (GPU-resident)" : ""}`, async () => {
        const g = new Gen(seeds[routine] + (resident ? 1000 : 0));
        let worst = 0;
        for (let run = 0; run < NUM_RUNS; run++) {
          const a = gemmArgs(g, routine, Arr);
          const got = await gemmRun(wg, device, a, Arr, resident);
          const { worst: f, untouched } = gemmFactor(got, a, Arr === Float64Array);
          const label = `run ${run}: ${a.layout} ${a.uplo || ""} ${a.transA}/${a.transB} m=${a.m} n=${a.n} k=${a.k}`;
          assert(f <= 1, `${label}: forward factor ${f} > 1`);
          assert(untouched, `${label}: an element outside the computed part changed`);
          worst = Math.max(worst, f);
        }
        assert(worst >= 0);
      });
    }
  }
  for (const [routine, r] of Object.entries(L1)) {
    for (const resident of [false, true]) {
      test(`fixtures: ${routine}, ${NUM_RUNS} random runs${resident ? " (GPU-resident)" : ""}`, async () => {
        const g = new Gen(seeds[routine] + (resident ? 1000 : 0));
        for (let run = 0; run < NUM_RUNS; run++) {
          const a = vecArgs(g, !!r.two);
          let got;
          if (resident) {
            const x = wg.GpuVector.from(device, a.x);
            const y = r.two ? wg.GpuVector.from(device, a.y) : null;
            try {
              got = await r.call(wg, device, a, x, y);
            } finally {
              x.destroy();
              if (y) y.destroy();
            }
          } else {
            got = await r.call(wg, device, a, a.x, a.y);
          }
          const m = r.metric(got, a);
          assert(m <= r.threshold, `run ${run}: n=${a.n} incx=${a.incx}: metric ${m} > ${r.threshold}`);
        }
      });
    }
  }
}
