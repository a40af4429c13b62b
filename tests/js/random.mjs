// randomFloat32Array / randomFloat64Array reproduce wgblas's seeded streams
// bit for bit (tests/golden/random_golden.json, written by the reference's
// src/random/random.mjs). randomTriangularFloat32Array draws from
// Math.random, so it is held to its properties: zero outside the triangle,
// the diagonal in [diagLow, diagHigh), the triangle in [low, high), and the
// reference's argument errors (src/random/random.mjs:28-60).
import { readFileSync } from "fs";
import { fileURLToPath } from "url";
import { dirname, join } from "path";
import { test, run, assert } from "./harness.mjs";
import { randomFloat32Array, randomFloat64Array, randomTriangularFloat32Array } from "../../wgblas_amd/js/src/random.mjs";
import * as viaSubpath from "../../wgblas_amd/js/index.mjs";

const here = dirname(fileURLToPath(import.meta.url));
const gold = JSON.parse(readFileSync(join(here, "..", "golden", "random_golden.json"), "utf8"));

for (const c of gold.cases) {
  test(`seed ${c.seed} n=${c.n} [${c.low}, ${c.high})`, () => {
    const f32 = new Uint32Array(randomFloat32Array(c.n, c.low, c.high, c.seed).buffer);
    const f64 = randomFloat64Array(c.n, c.low, c.high, c.seed);
    c.index.forEach((i, j) => {
      assert(f32[i] === c.f32_bits[j], `f32[${i}] bits ${f32[i]} != ${c.f32_bits[j]}`);
      assert(f64[i] === c.f64[j], `f64[${i}] ${f64[i]} != ${c.f64[j]}`);
    });
  });
}

test("unseeded draws stay in [low, high)", () => {
  const x = randomFloat64Array(1000, -2, 3);
  assert(x.every((v) => v >= -2 && v < 3));
});

// entry (i, j) of an n x n matrix stored with leading dimension lda
const at = (A, lda, layout, i, j) => (layout === "column-major" ? A[j * lda + i] : A[i * lda + j]);

for (const layout of ["row-major", "column-major"])
  for (const uplo of ["lower", "upper"])
    for (const [n, lda] of [[1, 1], [7, 7], [33, 40]]) {
      test(`randomTriangularFloat32Array ${uplo} ${layout} n=${n} lda=${lda}`, () => {
        const [low, high, dlo, dhi] = [-0.5, 0.25, 3, 4];
        const A = randomTriangularFloat32Array(n, lda, uplo, low, high, dlo, dhi, layout);
        assert(A instanceof Float32Array && A.length === n * lda, `length ${A.length}`);
        let offDiag = 0;
        for (let i = 0; i < n; i++)
          for (let j = 0; j < n; j++) {
            const v = at(A, lda, layout, i, j);
            if (i === j) assert(v >= Math.fround(dlo) && v <= Math.fround(dhi), `diag ${i}: ${v}`);
            else if (uplo === "lower" ? j < i : j > i) {
              assert(v >= Math.fround(low) && v <= Math.fround(high), `(${i},${j}) = ${v}`);
              offDiag += v !== 0;
            } else assert(Object.is(v, 0), `(${i},${j}) outside the triangle = ${v}`);
          }
        // padding past the n x n block stays zero
        for (let o = 0; o < n; o++)
          for (let p = n; p < lda; p++) assert(A[o * lda + p] === 0, `padding ${o}, ${p}`);
        if (n > 4) assert(offDiag > 0, "the triangle was filled");
      });
    }

test("randomTriangularFloat32Array defaults: lower, [-1, 1), diagonal [5, 15), row-major", () => {
  const A = randomTriangularFloat32Array(50, 50);
  for (let i = 0; i < 50; i++) {
    assert(A[i * 50 + i] >= 5 && A[i * 50 + i] < 15, `diag ${i}`);
    for (let j = i + 1; j < 50; j++) assert(A[i * 50 + j] === 0, `upper (${i},${j})`);
    for (let j = 0; j < i; j++) assert(A[i * 50 + j] >= -1 && A[i * 50 + j] < 1, `lower (${i},${j})`);
  }
});

test("randomTriangularFloat32Array argument errors", () => {
  const cases = [
    [() => randomTriangularFloat32Array(4, 4, "both"), "uplo must be 'lower' or 'upper'."],
    [() => randomTriangularFloat32Array(4, 4, "lower", -1, 1, 5, 15, "diagonal"),
     "layout must be 'row-major' or 'column-major'."],
    [() => randomTriangularFloat32Array(4, 3), "lda must be >= n."],
  ];
  for (const [fn, msg] of cases) {
    let got = null;
    try {
      fn();
    } catch (e) {
      got = e.message;
    }
    assert(got === msg, `expected "${msg}", got "${got}"`);
  }
});

test("the package root re-exports the random helpers", () => {
  assert(viaSubpath.randomTriangularFloat32Array === randomTriangularFloat32Array);
  assert(viaSubpath.randomFloat32Array === randomFloat32Array);
});

run();
