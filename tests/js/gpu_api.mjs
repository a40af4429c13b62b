// The device-handling and benchmark-mode checks of the JavaScript API on the
// GPU (init's device cache, gpuName, a second device with benchmark timing,
// foreign-device operands, cleanup of one device and of all), followed by
// every single-context case of parity_gpu.mjs on the first device.
import { test, run, assert, assertEqual } from "./harness.mjs";
import * as wg from "../../wgblas_amd/js/index.mjs";

let device;
let parity;  // parity_gpu.mjs, imported after the device case is registered

const exactEqual = (got, want, label) => {
  assertEqual(got.length, want.length, `${label}: length`);
  for (let i = 0; i < want.length; i++) assert(got[i] === want[i], `${label}: [${i}] = ${got[i]}, want ${want[i]}`);
};

// ------------------------------------------------------------------ device
test("init / gpuName / cleanup", async () => {
  device = await wg.init();
  parity.setParityDevice(device);
  assert(device instanceof wg.HipDevice);
  assert((await wg.init()) === device, "same options -> same device");
  const name = wg.gpuName(device);
  assert(/gfx950/.test(name.device), `arch ${name.device}`);
  const bench = await wg.init({ benchmark: true });
  assert(bench !== device);
  const x = wg.GpuVector.from(bench, new Float32Array([3, 4]));
  const r = await wg.snrm2(bench, 2, x, 1);
  assertEqual(r.nrm2, 5);
  assert(typeof r.gpuTimeMs === "number" && r.gpuTimeMs > 0, "gpuTimeMs in benchmark mode");
  let threw = false;
  try {
    await wg.snrm2(device, 2, x, 1);
  } catch (e) {
    threw = /different GPUDevice/.test(e.message);
  }
  assert(threw, "foreign-device operand rejected");
  x.destroy();
  wg.cleanup(bench);
  assert((await wg.init()) === device, "cleanup(one) keeps the others");
});

async function main() {
  // registers the single-context cases after the device case
  parity = await import("./parity_gpu.mjs");

  for (const [lA, lB] of [["row-major", "column-major"], ["column-major", "row-major"]])
    for (const trans of ["no-transpose", "transpose"])
      test(`ssyr2k GpuMatrix A ${lA}, B ${lB}, ${trans}, benchmark mode times the call`, async () => {
        const n = 90;
        const k = 33;
        const [r, c] = trans === "no-transpose" ? [n, k] : [k, n];
        const lda = (lA === "column-major" ? r : c) + 1;
        const ldb = (lB === "column-major" ? r : c) + 3;
        const a = { uplo: "upper", trans, n, k, alpha: 0.75, beta: -0.5, layoutA: lA, layoutB: lB, layoutC: "row-major",
          A: wg.randomFloat32Array((lA === "column-major" ? c : r) * lda, -1, 1, 74), lda,
          B: wg.randomFloat32Array((lB === "column-major" ? c : r) * ldb, -1, 1, 75), ldb,
          C: wg.randomFloat32Array(n * n, -1, 1, 76), ldc: n };
        const bench = await wg.init({ benchmark: true });
        const gA = wg.GpuMatrix.from(bench, a.A, r, c, lda, lA);
        const gB = wg.GpuMatrix.from(bench, a.B, r, c, ldb, lB);
        const gC = wg.GpuMatrix.from(bench, a.C, n, n, n, "row-major");
        try {
          const res = await wg.ssyr2k(bench, "upper", trans, n, k, 0.75, gA, lda, gB, ldb, -0.5, gC, n);
          assert(typeof res.gpuTimeMs === "number" && res.gpuTimeMs > 0, "one gpuTimeMs span for the call");
        } finally {
          gA.destroy();
          gB.destroy();
          gC.destroy();
          wg.cleanup(bench);
        }
      });

  test("sgemv alpha = 0, beta = 1 in benchmark mode reports this call's gpuTimeMs", async () => {
    const bench = await wg.init({ benchmark: true });
    const A = wg.GpuMatrix.from(bench, wg.randomFloat32Array(64 * 32, -1, 1, 77), 64, 32, 32);
    const x = wg.GpuVector.from(bench, wg.randomFloat32Array(32, -1, 1, 78));
    const y0 = wg.randomFloat32Array(64, -1, 1, 79);
    const y = wg.GpuVector.from(bench, y0);
    try {
      // a fresh benchmark device: no earlier timed call to fall back on
      const r = await wg.sgemv(bench, "no-transpose", 64, 32, 0, A, 32, x, 1, 1, y, 1);
      assert(typeof r.gpuTimeMs === "number" && r.gpuTimeMs >= 0, "gpuTimeMs present");
      exactEqual(await y.read(), y0, "y untouched");
    } finally {
      A.destroy();
      x.destroy();
      y.destroy();
      wg.cleanup(bench);
    }
  });

  test("cleanup() releases everything", async () => {
    wg.cleanup();
    let threw = false;
    try {
      wg.gpuName();
    } catch (e) {
      threw = /init\(\)/.test(e.message);
    }
    assert(threw);
  });

  await run();
}

main().catch((e) => {
  console.error(e);
  process.exitCode = 1;
});
