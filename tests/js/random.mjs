// randomFloat32Array / randomFloat64Array reproduce wgblas's seeded streams
// bit for bit (tests/golden/random_golden.json, written by the reference's
// src/random/random.mjs).
import { readFileSync } from "fs";
import { fileURLToPath } from "url";
import { dirname, join } from "path";
import { test, run, assert } from "./harness.mjs";
import { randomFloat32Array, randomFloat64Array } from "../../wgblas_amd/js/src/random.mjs";

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

run();
