// Writes tests/golden/random_golden.json: bit patterns of wgblas's seeded
// generators randomFloat32Array / randomFloat64Array
// (src/random/random.mjs:14-26), produced by the reference module itself.
// Run once in the build container (the reference is not on the GPU box):
//   node tests/golden/gen_random_golden.mjs /root/reference
import { writeFileSync } from "fs";
import { pathToFileURL, fileURLToPath } from "url";
import { dirname, join } from "path";

const refRoot = process.argv[2] || "/root/reference";
const here = dirname(fileURLToPath(import.meta.url));

async function main() {
  const mod = await import(pathToFileURL(join(refRoot, "src/random/random.mjs")).href);
  const cases = [];
  const specs = [
    { n: 16, low: -1, high: 1, seed: 0 },
    { n: 16, low: -1, high: 1, seed: 1 },
    { n: 16, low: -1, high: 1, seed: 2 },
    { n: 16, low: -1, high: 1, seed: 3 },
    { n: 16, low: -1, high: 1, seed: 4 },
    { n: 16, low: -5, high: 5, seed: 300 },
    { n: 16, low: 0, high: 1, seed: 4294967295 },
    { n: 16, low: -3.5, high: 12.25, seed: 123456789 },
    { n: 70000, low: -1, high: 1, seed: 100, sample: [0, 1, 4095, 65535, 65536, 69999] },
  ];
  for (const s of specs) {
    const f32 = mod.randomFloat32Array(s.n, s.low, s.high, s.seed);
    const f64 = mod.randomFloat64Array(s.n, s.low, s.high, s.seed);
    const bits = new Uint32Array(f32.buffer);
    const idx = s.sample || [...Array(s.n).keys()];
    cases.push({
      n: s.n, low: s.low, high: s.high, seed: s.seed, index: idx,
      f32_bits: idx.map((i) => bits[i]),
      f64: idx.map((i) => f64[i]),
    });
  }
  writeFileSync(join(here, "random_golden.json"), JSON.stringify({ source: "src/random/random.mjs", cases }, null, 1) + "\n");
  console.log(`wrote ${cases.length} cases`);
}
main().catch((e) => { console.error(e); process.exit(1); });
