// Argument-validation contract of the JavaScript API, driven by the
// reference's own parameter specs (tests/golden/validation_params/*.json,
// copied data of wgblas's tests/validation/params). For every routine on the
// path, each spec's `invalid` entries are substituted one at a time into a
// valid baseline call and must throw an Error whose message contains the
// spec's `error` text; with --gpu, each `edge` entry must run without
// throwing. The baseline assembly follows the behaviour of wgblas's
// tests/helpers/validation.js (loadParam, runValidation, minimal/tooShort
// array sizing); the spec composition per routine follows wgblas's
// tests/<routine>/src/test.<routine>.js.
//
//   node tests/js/validation.mjs          # invalid cases, no GPU needed
//   node tests/js/validation.mjs --gpu    # invalid + edge cases on the GPU,
//                                         # plus resident_gpu.mjs,
//                                         # parity_gpu.mjs and fixtures_gpu.mjs
import { readFileSync } from "fs";
import { fileURLToPath } from "url";
import { dirname, join } from "path";
import { test, run, assertRejects } from "./harness.mjs";
import { registerResidentTests, registerCleanupTest } from "./resident_gpu.mjs";
import * as wg from "../../wgblas_amd/js/index.mjs";

const here = dirname(fileURLToPath(import.meta.url));
const PARAMS = join(here, "..", "golden", "validation_params");
const GPU = process.argv.includes("--gpu");

function loadParam(name) {
  if (name.endsWith("64")) return derive64(loadParam(name.slice(0, -2)));
  return JSON.parse(readFileSync(join(PARAMS, `${name}.json`), "utf8"));
}

// The Float64Array variant of a float32 spec: same cases, f64 wording, and a
// GpuMatrix / GpuVector-of-the-wrong-dtype case for matrix / vector specs.
function derive64(base) {
  const isArray = base.type !== "float";
  const isMatrix = (base.dependsOn || []).some((d) => d.startsWith("ld"));
  const invalid = (base.invalid || []).map((e) =>
    Object.assign({}, e, { error: typeof e.error === "string" ? e.error.replace("Float32Array", "Float64Array") : e.error }));
  if (base.type === "float32array" && isMatrix)
    invalid.push({ scenario: "wrongDtypeGpuMatrix", error: "must be a Float64Array-backed GpuMatrix", label: "GpuMatrix of Float32Array" });
  if (base.type === "float32array" && !isMatrix)
    invalid.push({ scenario: "wrongDtypeGpuVector", error: "must be a Float64Array-backed GpuVector", label: "GpuVector of Float32Array" });
  return Object.assign({}, base, { type: isArray ? "float64array" : "float64", invalid });
}

const SPECIALS = { NaN: NaN, Infinity: Infinity, "-Infinity": -Infinity, null: null, undefined: undefined,
  string: "100", array: [], object: {}, number: 42 };

const ctorOf = (type) => (type === "float64array" ? Float64Array : Float32Array);

// Logical {outer, inner} of a matrix param from its dependsOn (the cases the
// path needs: a level-3 operand with its own trans flag, or a plain m x n /
// n x n matrix).
function matrixShape(dependsOn, dims) {
  const deps = new Set(dependsOn || []);
  const transKey = (dependsOn || []).find((d) => d.startsWith("trans"));
  const cm = dims.layout === "column-major";
  if (transKey && deps.has("k")) {
    const [d1, d2] = dependsOn.filter((d) => d === "m" || d === "n" || d === "k");
    const rows = cm ? dims[d2] : dims[d1];
    const cols = cm ? dims[d1] : dims[d2];
    const noTrans = (dims[transKey] || "no-transpose") === "no-transpose";
    return noTrans ? { outer: rows, inner: cols } : { outer: cols, inner: rows };
  }
  if (deps.has("side")) {
    const order = (dims.side || "left") === "left" ? dims.m : dims.n;
    return { outer: order, inner: order };
  }
  if (deps.has("m") && deps.has("n")) return cm ? { outer: dims.n, inner: dims.m } : { outer: dims.m, inner: dims.n };
  if (deps.has("n")) return { outer: dims.n, inner: dims.n };
  return null;
}

function minLength(dependsOn, dims) {
  const ldKey = (dependsOn || []).find((d) => d.startsWith("ld"));
  if (ldKey) {
    const s = matrixShape(dependsOn, dims);
    if (s) return Math.max(0, (s.outer - 1) * dims[ldKey] + s.inner);
  }
  const isX = (dependsOn || []).includes("incx");
  const inc = isX ? (dims.incx || 1) : (dims.incy || 1);
  let len = dims.n === undefined ? 4 : dims.n;
  // sgemv's x / y: the active length follows trans (row-major frame); the
  // same specs serve sdot / ddot, which have no m
  if ((dependsOn || []).includes("trans") && (dependsOn || []).includes("m") && dims.m !== undefined) {
    const noTrans = (dims.trans || "no-transpose") === "no-transpose";
    len = noTrans === isX ? dims.n : dims.m;
  } else if ((dependsOn || []).includes("m") && !(dependsOn || []).includes("n")) {
    // a vector sized by m alone (sger's x)
    len = dims.m;
  }
  return (len - 1) * inc + 1;
}

function resolve(entry, name, spec, baselines, device) {
  if ("scenario" in entry) {
    if (entry.scenario === "wrongDtypeGpuMatrix") {
      const data = new Float32Array(16).fill(1);
      return wg.GpuMatrix.from(device, data, 2, 2, 2, baselines.layout || "row-major");
    }
    if (entry.scenario === "wrongDtypeGpuVector")
      return wg.GpuVector.from(device, new Float32Array(minLength(spec.dependsOn, baselines)).fill(1));
    const len = minLength(spec.dependsOn, baselines);
    const Ctor = ctorOf(spec.type);
    if (entry.scenario === "minimal") return new Ctor(len).fill(1);
    if (entry.scenario === "tooShort") return new Ctor(Math.max(0, len - 1)).fill(1);
    throw new Error(`unknown scenario ${entry.scenario}`);
  }
  if ("value" in entry) {
    if (Array.isArray(entry.value) && /array$/.test(spec.type || "")) return new (ctorOf(spec.type))(entry.value);
    return entry.value;
  }
  return SPECIALS[entry.special];
}

function baselinesOf(specs, device) {
  const b = { device };
  for (const [name, spec] of Object.entries(specs)) {
    if (!("baseline" in spec)) continue;
    b[name] = Array.isArray(spec.baseline) ? new (ctorOf(spec.type))(spec.baseline) : spec.baseline;
  }
  for (const [name, spec] of Object.entries(specs)) {
    if (b[name] !== undefined || !/array$/.test(spec.type || "")) continue;
    const deps = new Set(spec.dependsOn || []);
    const dims = Object.assign({}, b);
    // sized so the baseline survives every leading-dimension / stride edge case
    if (deps.has("lda") && specs.lda && specs.lda.range) dims.lda = specs.lda.range.max;
    if (deps.has("incx") && specs.incx && specs.incx.range) dims.incx = specs.incx.range.max;
    if (deps.has("incy") && specs.incy && specs.incy.range) dims.incy = specs.incy.range.max;
    b[name] = new (ctorOf(spec.type))(minLength(spec.dependsOn, dims)).fill(1);
  }
  return b;
}

// Arrays whose shape depends on a parameter an edge case changes (trans,
// side, m, ...) are rebuilt for that case at the minimal valid length, with
// leading dimensions and strides at the top of their ranges as in the
// baselines.
function resized(specs, args, changed) {
  const out = Object.assign({}, args);
  for (const [name, spec] of Object.entries(specs)) {
    if (name === changed || "baseline" in spec || !/array$/.test(spec.type || "")) continue;
    if (!(spec.dependsOn || []).includes(changed)) continue;
    const deps = new Set(spec.dependsOn || []);
    const dims = Object.assign({}, out);
    for (const k of ["lda", "incx", "incy"])
      if (deps.has(k) && k !== changed && specs[k] && specs[k].range) dims[k] = specs[k].range.max;
    out[name] = new (ctorOf(spec.type))(Math.max(1, minLength(spec.dependsOn, dims))).fill(1);
  }
  return out;
}

function register(routine, specs, call, device) {
  const baselines = baselinesOf(specs, device);
  for (const [name, spec] of Object.entries(specs)) {
    for (const entry of spec.invalid || []) {
      if (!GPU && /^wrongDtype/.test(entry.scenario || "")) continue;
      test(`${routine} ${name} invalid: ${entry.label || JSON.stringify(entry)}`, async () => {
        const args = Object.assign({}, baselines);
        args[name] = resolve(entry, name, spec, baselines, device);
        try {
          await assertRejects(() => call(args), entry.error);
        } finally {
          if (args[name] instanceof wg.GpuMatrix || args[name] instanceof wg.GpuVector) args[name].destroy();
        }
      });
    }
    // Edge cases must pass argument validation. On the GPU they run; on the
    // CPU the device is a released handle, so a call that gets as far as the
    // device fails with exactly that error, and any other error is a
    // validation (shape) failure.
    for (const entry of spec.edge || []) {
      test(`${routine} ${name} edge: ${entry.label || JSON.stringify(entry)}`, async () => {
        const args = resized(specs, Object.assign({}, baselines, { [name]: resolve(entry, name, spec, baselines, device) }),
          name);
        try {
          await call(args);
        } catch (e) {
          if (!GPU && /released by cleanup/.test(String(e && e.message))) return;
          throw e;
        }
      });
    }
  }
}

function nWithNegative(error) {
  const n = loadParam("n");
  return Object.assign({}, n, {
    baseline: 2,
    edge: n.edge.filter((e) => e.value !== -1),
    invalid: n.invalid.concat([{ value: -1, error, label: "negative" }]),
  });
}

function gemmSpecs(f64) {
  const ld = loadParam("ld");
  const A = f64 ? loadParam("A64") : loadParam("A");
  const lvl3 = loadParam("A")["level-3"];
  const aSpec = Object.assign({}, A, {
    dependsOn: lvl3.dependsOn,
    edge: lvl3.edge,
    invalid: lvl3.invalid
      .map((e) => Object.assign({}, e, { error: f64 ? e.error.replace("Float32Array", "Float64Array") : e.error }))
      .concat(f64 ? A.invalid.filter((e) => e.scenario === "wrongDtypeGpuMatrix") : []),
  });
  return {
    device: loadParam("device"),
    transA: loadParam("trans"),
    transB: loadParam("trans"),
    layout: loadParam("layout"),
    m: Object.assign({}, loadParam("m"), { baseline: 2 }),
    n: nWithNegative("m, n, and k must be non-negative"),
    k: loadParam("k"),
    alpha: loadParam("alpha"),
    beta: loadParam("beta"),
    A: aSpec,
    lda: ld,
    B: f64 ? loadParam("B64") : loadParam("B"),
    ldb: ld,
    C: f64 ? loadParam("C64") : loadParam("C"),
    ldc: ld,
  };
}

async function main() {
  const device = GPU ? await wg.init() : Object.assign(Object.create(wg.HipDevice.prototype), { _ctx: null });
  const g = gemmSpecs(false);
  register("sgemm", g, (a) => wg.sgemm(a.device, a.transA, a.transB, a.m, a.n, a.k, a.alpha, a.A, a.lda, a.B, a.ldb, a.beta, a.C, a.ldc, a.layout), device);
  register("sgemmtr", Object.assign({ uplo: loadParam("uplo") }, g),
    (a) => wg.sgemmtr(a.device, a.uplo, a.transA, a.transB, a.m, a.n, a.k, a.alpha, a.A, a.lda, a.B, a.ldb, a.beta, a.C, a.ldc, a.layout), device);
  register("dgemm", gemmSpecs(true),
    (a) => wg.dgemm(a.device, a.transA, a.transB, a.m, a.n, a.k, a.alpha, a.A, a.lda, a.B, a.ldb, a.beta, a.C, a.ldc, a.layout), device);
  const A = loadParam("A");
  register("ssyrk", {
    device: loadParam("device"),
    uplo: loadParam("uplo"),
    trans: loadParam("trans"),
    layout: loadParam("layout"),
    n: nWithNegative("must be non-negative"),
    k: loadParam("k"),
    alpha: loadParam("alpha"),
    beta: loadParam("beta"),
    A: Object.assign({}, A, A["level-3"], { dependsOn: ["n", "k", "lda", "trans"] }),
    lda: loadParam("ld"),
    C: Object.assign({}, loadParam("C"), { dependsOn: ["n", "ldc"] }),
    ldc: loadParam("ld"),
  }, (a) => wg.ssyrk(a.device, a.uplo, a.trans, a.n, a.k, a.alpha, a.A, a.lda, a.beta, a.C, a.ldc, a.layout), device);
  register("dgemmtr", Object.assign({ uplo: loadParam("uplo") }, gemmSpecs(true)),
    (a) => wg.dgemmtr(a.device, a.uplo, a.transA, a.transB, a.m, a.n, a.k, a.alpha, a.A, a.lda, a.B, a.ldb, a.beta, a.C, a.ldc, a.layout), device);
  // dsyrk: wgblas's tests/dsyrk/src/test.dsyrk.js composition (A64 with the
  // level-3 edge/invalid cases in f64 wording plus the wrong-dtype GpuMatrix).
  const A64 = loadParam("A64");
  register("dsyrk", {
    device: loadParam("device"),
    uplo: loadParam("uplo"),
    trans: loadParam("trans"),
    layout: loadParam("layout"),
    n: nWithNegative("must be non-negative"),
    k: loadParam("k"),
    alpha: loadParam("alpha"),
    beta: loadParam("beta"),
    A: Object.assign({}, A64, {
      edge: A["level-3"].edge,
      invalid: A["level-3"].invalid
        .map((e) => Object.assign({}, e, { error: e.error.replace("Float32Array", "Float64Array") }))
        .concat(A64.invalid.filter((e) => e.scenario === "wrongDtypeGpuMatrix")),
      dependsOn: ["n", "k", "lda", "trans"],
    }),
    lda: loadParam("ld"),
    C: Object.assign({}, loadParam("C64"), { dependsOn: ["n", "ldc"] }),
    ldc: loadParam("ld"),
  }, (a) => wg.dsyrk(a.device, a.uplo, a.trans, a.n, a.k, a.alpha, a.A, a.lda, a.beta, a.C, a.ldc, a.layout), device);
  // level 3 on the GEMM: wgblas's tests/{ssyr2k,ssymm,strmm,strsm}/src/test.*.js
  // compositions.
  register("ssyr2k", {
    device: loadParam("device"),
    uplo: loadParam("uplo"),
    trans: loadParam("trans"),
    layout: loadParam("layout"),
    n: nWithNegative("must be non-negative"),
    k: loadParam("k"),
    alpha: loadParam("alpha"),
    beta: loadParam("beta"),
    A: Object.assign({}, A, A["level-3"], { dependsOn: ["n", "k", "lda", "trans"] }),
    lda: loadParam("ld"),
    B: Object.assign({}, loadParam("B"), { dependsOn: ["n", "k", "ldb", "trans"] }),
    ldb: loadParam("ld"),
    C: Object.assign({}, loadParam("C"), { dependsOn: ["n", "ldc"] }),
    ldc: loadParam("ld"),
  }, (a) => wg.ssyr2k(a.device, a.uplo, a.trans, a.n, a.k, a.alpha, a.A, a.lda, a.B, a.ldb, a.beta, a.C, a.ldc,
    a.layout), device);
  register("ssymm", {
    device: loadParam("device"),
    side: loadParam("side"),
    uplo: loadParam("uplo"),
    layout: loadParam("layout"),
    m: Object.assign({}, loadParam("m"), { baseline: 2 }),
    n: nWithNegative("must be non-negative"),
    alpha: loadParam("alpha"),
    beta: loadParam("beta"),
    A: Object.assign({}, A, { dependsOn: ["m", "n", "lda", "side"] }),
    lda: loadParam("ld"),
    B: Object.assign({}, loadParam("B"), { dependsOn: ["m", "n", "ldb"] }),
    ldb: loadParam("ld"),
    C: loadParam("C"),
    ldc: loadParam("ld"),
  }, (a) => wg.ssymm(a.device, a.side, a.uplo, a.m, a.n, a.alpha, a.A, a.lda, a.B, a.ldb, a.beta, a.C, a.ldc,
    a.layout), device);
  for (const r of ["strmm", "strsm"])
    register(r, {
      device: loadParam("device"),
      side: loadParam("side"),
      uplo: loadParam("uplo"),
      transA: loadParam("trans"),
      diag: loadParam("diag"),
      layout: loadParam("layout"),
      m: Object.assign({}, loadParam("m"), { baseline: 2 }),
      n: nWithNegative("must be non-negative"),
      alpha: loadParam("alpha"),
      A: Object.assign({}, A, { dependsOn: ["m", "n", "lda", "side"] }),
      lda: loadParam("ld"),
      B: Object.assign({}, loadParam("B"), { dependsOn: ["m", "n", "ldb"] }),
      ldb: loadParam("ld"),
    }, (a) => wg[r](a.device, a.side, a.uplo, a.transA, a.diag, a.m, a.n, a.alpha, a.A, a.lda, a.B, a.ldb,
      a.layout), device);
  // fp64 level 3: wgblas's tests/{dsyr2k,dsymm,dtrmm}/src/test.*.js
  // compositions (A64 / B64 / C64; dsyr2k's A with the level-3 cases in f64
  // wording, as dsyrk's).
  register("dsyr2k", {
    device: loadParam("device"),
    uplo: loadParam("uplo"),
    trans: loadParam("trans"),
    layout: loadParam("layout"),
    n: nWithNegative("must be non-negative"),
    k: loadParam("k"),
    alpha: loadParam("alpha"),
    beta: loadParam("beta"),
    A: Object.assign({}, A64, {
      edge: A["level-3"].edge,
      invalid: A["level-3"].invalid
        .map((e) => Object.assign({}, e, { error: e.error.replace("Float32Array", "Float64Array") }))
        .concat(A64.invalid.filter((e) => e.scenario === "wrongDtypeGpuMatrix")),
      dependsOn: ["n", "k", "lda", "trans"],
    }),
    lda: loadParam("ld"),
    B: Object.assign({}, loadParam("B64"), { dependsOn: ["n", "k", "ldb", "trans"] }),
    ldb: loadParam("ld"),
    C: Object.assign({}, loadParam("C64"), { dependsOn: ["n", "ldc"] }),
    ldc: loadParam("ld"),
  }, (a) => wg.dsyr2k(a.device, a.uplo, a.trans, a.n, a.k, a.alpha, a.A, a.lda, a.B, a.ldb, a.beta, a.C, a.ldc,
    a.layout), device);
  register("dsymm", {
    device: loadParam("device"),
    side: loadParam("side"),
    uplo: loadParam("uplo"),
    layout: loadParam("layout"),
    m: Object.assign({}, loadParam("m"), { baseline: 2 }),
    n: nWithNegative("must be non-negative"),
    alpha: loadParam("alpha"),
    beta: loadParam("beta"),
    A: Object.assign({}, A64, { dependsOn: ["m", "n", "lda", "side"] }),
    lda: loadParam("ld"),
    B: Object.assign({}, loadParam("B64"), { dependsOn: ["m", "n", "ldb"] }),
    ldb: loadParam("ld"),
    C: loadParam("C64"),
    ldc: loadParam("ld"),
  }, (a) => wg.dsymm(a.device, a.side, a.uplo, a.m, a.n, a.alpha, a.A, a.lda, a.B, a.ldb, a.beta, a.C, a.ldc,
    a.layout), device);
  register("dtrmm", {
    device: loadParam("device"),
    side: loadParam("side"),
    uplo: loadParam("uplo"),
    transA: loadParam("trans"),
    diag: loadParam("diag"),
    layout: loadParam("layout"),
    m: Object.assign({}, loadParam("m"), { baseline: 2 }),
    n: nWithNegative("must be non-negative"),
    alpha: loadParam("alpha"),
    A: Object.assign({}, A64, { dependsOn: ["m", "n", "lda", "side"] }),
    lda: loadParam("ld"),
    B: Object.assign({}, loadParam("B64"), { dependsOn: ["m", "n", "ldb"] }),
    ldb: loadParam("ld"),
  }, (a) => wg.dtrmm(a.device, a.side, a.uplo, a.transA, a.diag, a.m, a.n, a.alpha, a.A, a.lda, a.B, a.ldb,
    a.layout), device);
  // sgemv: wgblas's tests/sgemv/src/test.sgemv.js composition
  const nS = loadParam("n");
  register("sgemv", {
    device: loadParam("device"),
    trans: loadParam("trans"),
    m: loadParam("m"),
    n: Object.assign({}, nS, {
      edge: nS.edge.filter((e) => e.value !== -1),
      invalid: nS.invalid.concat([{ value: -1, error: "n must be non-negative", label: "negative" }]),
    }),
    alpha: loadParam("alpha"),
    beta: loadParam("beta"),
    lda: loadParam("lda"),
    A: loadParam("A"),
    x: loadParam("x"),
    incx: loadParam("incx"),
    y: loadParam("y"),
    incy: loadParam("incy"),
    layout: loadParam("layout"),
  }, (a) => wg.sgemv(a.device, a.trans, a.m, a.n, a.alpha, a.A, a.lda, a.x, a.incx, a.beta, a.y, a.incy,
    a.layout), device);
  // dgemv: wgblas's tests/dgemv/src/test.dgemv.js composition (alpha64 /
  // beta64 / A64 / x64 / y64)
  register("dgemv", {
    device: loadParam("device"),
    trans: loadParam("trans"),
    m: loadParam("m"),
    n: Object.assign({}, nS, {
      edge: nS.edge.filter((e) => e.value !== -1),
      invalid: nS.invalid.concat([{ value: -1, error: "n must be non-negative", label: "negative" }]),
    }),
    alpha: loadParam("alpha64"),
    beta: loadParam("beta64"),
    lda: loadParam("lda"),
    A: loadParam("A64"),
    x: loadParam("x64"),
    incx: loadParam("incx"),
    y: loadParam("y64"),
    incy: loadParam("incy"),
    layout: loadParam("layout"),
  }, (a) => wg.dgemv(a.device, a.trans, a.m, a.n, a.alpha, a.A, a.lda, a.x, a.incx, a.beta, a.y, a.incy,
    a.layout), device);
  // sger / dger: wgblas's tests/sger/src/test.sger.js and test.dger.js
  // compositions (x sized by m, y by n; dger with the 64-bit specs)
  for (const [r, f64] of [["sger", false], ["dger", true]]) {
    const v = (name) => loadParam(f64 ? name + "64" : name);
    register(r, {
      device: loadParam("device"),
      m: loadParam("m"),
      n: Object.assign({}, nS, {
        edge: nS.edge.filter((e) => e.value !== -1),
        invalid: nS.invalid.concat([{ value: -1, error: "n must be non-negative", label: "negative" }]),
      }),
      alpha: v("alpha"),
      x: Object.assign({}, v("x"), { dependsOn: ["m", "incx"] }),
      incx: loadParam("incx"),
      y: Object.assign({}, v("y"), { dependsOn: ["n", "incy"] }),
      incy: loadParam("incy"),
      A: v("A"),
      lda: loadParam("lda"),
      layout: loadParam("layout"),
    }, (a) => wg[r](a.device, a.m, a.n, a.alpha, a.x, a.incx, a.y, a.incy, a.A, a.lda, a.layout), device);
  }
  // ssyr / dsyr, ssyr2 / dsyr2: wgblas's tests/{ssyr,dsyr,ssyr2,dsyr2}/src
  // compositions (x and y sized by n, A n x n)
  for (const [r, f64, two] of [["ssyr", false, false], ["dsyr", true, false], ["ssyr2", false, true],
    ["dsyr2", true, true]]) {
    const v = (name) => loadParam(f64 ? name + "64" : name);
    const specs = {
      device: loadParam("device"),
      uplo: loadParam("uplo"),
      n: Object.assign({}, nS, {
        edge: nS.edge.filter((e) => e.value !== -1),
        invalid: nS.invalid.concat([{ value: -1, error: "n must be non-negative", label: "negative" }]),
      }),
      alpha: v("alpha"),
      x: Object.assign({}, v("x"), { dependsOn: ["n", "incx"] }),
      incx: loadParam("incx"),
      A: Object.assign({}, v("A"), { dependsOn: ["n", "lda"] }),
      lda: loadParam("lda"),
      layout: loadParam("layout"),
    };
    if (two) {
      specs.y = Object.assign({}, v("y"), { dependsOn: ["n", "incy"] });
      specs.incy = loadParam("incy");
    }
    register(r, specs, two
      ? (a) => wg[r](a.device, a.uplo, a.n, a.alpha, a.x, a.incx, a.y, a.incy, a.A, a.lda, a.layout)
      : (a) => wg[r](a.device, a.uplo, a.n, a.alpha, a.x, a.incx, a.A, a.lda, a.layout), device);
  }
  // ssymv / dsymv: wgblas's tests/ssymv/src/test.ssymv.js composition (dsymv
  // with the 64-bit specs)
  for (const [r, f64] of [["ssymv", false], ["dsymv", true]]) {
    const v = (name) => loadParam(f64 ? name + "64" : name);
    register(r, {
      device: loadParam("device"),
      uplo: loadParam("uplo"),
      n: Object.assign({}, nS, {
        edge: nS.edge.filter((e) => e.value !== -1),
        invalid: nS.invalid.concat([{ value: -1, error: "n must be non-negative", label: "negative" }]),
      }),
      alpha: v("alpha"),
      A: Object.assign({}, v("A"), { dependsOn: ["n", "lda"] }),
      lda: loadParam("lda"),
      x: Object.assign({}, v("x"), { dependsOn: ["n", "incx"] }),
      incx: loadParam("incx"),
      beta: v("beta"),
      y: Object.assign({}, v("y"), { dependsOn: ["n", "incy"] }),
      incy: loadParam("incy"),
      layout: loadParam("layout"),
    }, (a) => wg[r](a.device, a.uplo, a.n, a.alpha, a.A, a.lda, a.x, a.incx, a.beta, a.y, a.incy, a.layout),
    device);
  }
  // strmv / dtrmv: wgblas's tests/strmv/src/test.strmv.js composition
  // (dtrmv with the 64-bit specs)
  for (const [r, f64] of [["strmv", false], ["dtrmv", true]]) {
    const v = (name) => loadParam(f64 ? name + "64" : name);
    register(r, {
      device: loadParam("device"),
      uplo: loadParam("uplo"),
      trans: loadParam("trans"),
      diag: loadParam("diag"),
      n: Object.assign({}, nS, {
        edge: nS.edge.filter((e) => e.value !== -1),
        invalid: nS.invalid.concat([{ value: -1, error: "n must be non-negative", label: "negative" }]),
      }),
      A: Object.assign({}, v("A"), { dependsOn: ["n", "lda"] }),
      lda: loadParam("lda"),
      x: Object.assign({}, v("x"), { dependsOn: ["n", "incx"] }),
      incx: loadParam("incx"),
      y: Object.assign({}, v("y"), { dependsOn: ["n", "incy"] }),
      incy: loadParam("incy"),
      layout: loadParam("layout"),
    }, (a) => wg[r](a.device, a.uplo, a.trans, a.diag, a.n, a.A, a.lda, a.x, a.incx, a.y, a.incy, a.layout),
    device);
  }
  register("sdot", {
    device: loadParam("device"), n: loadParam("n"), incx: loadParam("incx"), incy: loadParam("incy"),
    x: loadParam("x"), y: loadParam("y"),
  }, (a) => wg.sdot(a.device, a.n, a.x, a.incx, a.y, a.incy), device);
  for (const r of ["sasum", "snrm2", "isamax"])
    register(r, { device: loadParam("device"), n: loadParam("n"), incx: loadParam("incx"), x: loadParam("x") },
      (a) => wg[r](a.device, a.n, a.x, a.incx), device);
  // fp64 level 1: wgblas's tests/{ddot,dasum,dnrm2,idamax}/src/test.*.js
  // compositions (x64 / y64 derived from the f32 specs).
  register("ddot", {
    device: loadParam("device"), n: loadParam("n"), incx: loadParam("incx"), incy: loadParam("incy"),
    x: loadParam("x64"), y: loadParam("y64"),
  }, (a) => wg.ddot(a.device, a.n, a.x, a.incx, a.y, a.incy), device);
  for (const r of ["dasum", "dnrm2", "idamax"])
    register(r, { device: loadParam("device"), n: loadParam("n"), incx: loadParam("incx"), x: loadParam("x64") },
      (a) => wg[r](a.device, a.n, a.x, a.incx), device);
  if (GPU) {
    registerResidentTests(wg, device);
    // the JS API's single-context parity cases (fixtures, regressions,
    // residency) on the same device
    const parity = await import("./parity_gpu.mjs");
    parity.setParityDevice(device);
    // random fixtures in the shape of the reference's runFixtures
    const fixtures = await import("./fixtures_gpu.mjs");
    fixtures.registerFixtureTests(wg, device);
    registerCleanupTest(wg, device);
  }
  await run();
  if (GPU) wg.cleanup();
}

main().catch((e) => {
  console.error(e);
  process.exitCode = 1;
});
