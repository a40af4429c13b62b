// CPU check of fixtures_gpu.mjs's checker: its runs and metrics, driven
// through CPU stand-ins for the routines and the GpuMatrix / GpuVector
// classes. With the stand-ins computing each result in float64 and rounding
// it to the array type once, every fixture must pass; with one mistake
// planted in a stand-in (the mode argument), that routine's fixtures must
// fail. No GPU and no addon are involved.
//
//   node tests/js/fixtures_selfcheck.mjs good
//   node tests/js/fixtures_selfcheck.mjs <mode>   # one planted mistake, see MODES
import { run } from "./harness.mjs";
import { registerFixtureTests } from "./fixtures_gpu.mjs";

const mode = process.argv[2] || "good";
// mode -> what the stand-in gets wrong
const MODES = {
  good: "nothing",
  beta: "sgemm ignores beta C",
  trans: "sgemm reads op(A) as A",
  tri: "sgemmtr also writes the other triangle",
  syrk: "ssyrk reads op(A) op(A)^T as op(A)^T op(A)",
  dgemm_round: "dgemm rounds its result to float32",
  dot: "sdot skips its last product",
  asum: "sasum sums signed values",
  nrm2: "snrm2 skips its last element",
  amax: "isamax compares signed values instead of magnitudes",
};
if (!(mode in MODES)) throw new Error(`unknown mode ${mode}`);

class FakeMatrix {
  constructor(data, rows, cols, ld, layout) {
    this.data = data.slice();
    this.rows = rows;
    this.cols = cols;
    this.lda = ld;
    this.layout = layout;
  }
  static from(device, data, rows, cols, ld, layout = "row-major") {
    return new FakeMatrix(data, rows, cols, ld, layout);
  }
  async read() {
    const cm = this.layout === "column-major";
    const outer = cm ? this.cols : this.rows;
    const inner = cm ? this.rows : this.cols;
    const out = new this.data.constructor(outer * inner);
    for (let o = 0; o < outer; o++) out.set(this.data.subarray(o * this.lda, o * this.lda + inner), o * inner);
    return out;
  }
  destroy() {}
}

class FakeVector {
  constructor(data) {
    this.data = data.slice();
  }
  static from(device, data) {
    return new FakeVector(data);
  }
  destroy() {}
}

const raw = (X) => (X instanceof FakeMatrix || X instanceof FakeVector ? X.data : X);
const at = (M, ld, layout, r, c) => (layout === "column-major" ? M[c * ld + r] : M[r * ld + c]);
const opAt = (M, ld, layout, trans, r, c) =>
  trans === "transpose" ? at(M, ld, layout, c, r) : at(M, ld, layout, r, c);

function gemm(routine, uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, layout) {
  const cm = layout === "column-major";
  const out = raw(C).slice();
  const round = routine === "dgemm" && mode !== "dgemm_round" ? (x) => x : Math.fround;
  const tA = routine === "sgemm" && mode === "trans" ? "no-transpose" : transA;
  for (let i = 0; i < m; i++)
    for (let j = 0; j < n; j++) {
      const inside = !uplo || (uplo === "lower" ? i >= j : i <= j);
      if (!inside && !(routine === "sgemmtr" && mode === "tri")) continue;
      let s = 0;
      // (the planted transpose mistake may read past A: undefined -> NaN)
      for (let p = 0; p < k; p++) s += opAt(raw(A), lda, layout, tA, i, p) * opAt(raw(B), ldb, layout, transB, p, j);
      const q = cm ? j * ldc + i : i * ldc + j;
      const withC = routine === "sgemm" && mode === "beta" ? 0 : beta * out[q];
      out[q] = round(alpha * s + withC);
    }
  if (C instanceof FakeMatrix) {
    C.data = out;
    return {};
  }
  return { C: out };
}

const vec = (X) => raw(X);
const wg = {
  GpuMatrix: FakeMatrix,
  GpuVector: FakeVector,
  async sgemm(d, tA, tB, m, n, k, al, A, lda, B, ldb, be, C, ldc, layout) {
    return gemm("sgemm", null, tA, tB, m, n, k, al, A, lda, B, ldb, be, C, ldc, layout);
  },
  async dgemm(d, tA, tB, m, n, k, al, A, lda, B, ldb, be, C, ldc, layout) {
    return gemm("dgemm", null, tA, tB, m, n, k, al, A, lda, B, ldb, be, C, ldc, layout);
  },
  async sgemmtr(d, uplo, tA, tB, m, n, k, al, A, lda, B, ldb, be, C, ldc, layout) {
    return gemm("sgemmtr", uplo, tA, tB, m, n, k, al, A, lda, B, ldb, be, C, ldc, layout);
  },
  async ssyrk(d, uplo, trans, n, k, al, A, lda, be, C, ldc, layout) {
    let tA = trans;
    if (mode === "syrk") tA = trans === "transpose" ? "no-transpose" : "transpose";
    const tB = tA === "transpose" ? "no-transpose" : "transpose";
    // the planted mistake reads A with the other shape: keep it in bounds
    // by reading zeros where that shape leaves the array
    const AA = raw(A);
    const guard = new Proxy(AA, { get: (t, p) => (typeof p === "string" && /^\d+$/.test(p) && +p >= t.length ? 0 : t[p]) });
    return gemm("ssyrk", uplo, tA, tB, n, n, k, al, guard, lda, guard, lda, be, C, ldc, layout);
  },
  async sdot(d, n, x, incx, y, incy) {
    let s = 0;
    const last = mode === "dot" ? n - 1 : n;
    for (let i = 0; i < last; i++) s += vec(x)[i * incx] * vec(y)[i * incy];
    return { dot: Math.fround(s) };
  },
  async sasum(d, n, x, incx) {
    let s = 0;
    for (let i = 0; i < n; i++) s += mode === "asum" ? vec(x)[i * incx] : Math.abs(vec(x)[i * incx]);
    return { asum: Math.fround(mode === "asum" ? Math.abs(s) : s) };
  },
  async snrm2(d, n, x, incx) {
    let s = 0;
    const last = mode === "nrm2" ? n - 1 : n;
    for (let i = 0; i < last; i++) s += vec(x)[i * incx] ** 2;
    return { nrm2: Math.fround(Math.sqrt(s)) };
  },
  async isamax(d, n, x, incx) {
    let best = 0;
    const mag = mode === "amax" ? (v) => v : Math.abs;
    for (let i = 1; i < n; i++) if (mag(vec(x)[i * incx]) > mag(vec(x)[best * incx])) best = i;
    return { index: best };
  },
};

console.log(`mode ${mode}: ${MODES[mode]}`);
registerFixtureTests(wg, {});
run();
