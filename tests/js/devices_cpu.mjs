// The JS layer's device handling on the CPU, against the host-memory stand-in
// stub_addon.cjs (run with WGBLAS_HIP_ADDON pointing at it): wgblas's init()
// cache keyed by the resolved options, cleanup(one) releasing only that
// device, cleanup() releasing all, gpuName on the first device, operands of
// another device rejected, GpuVector / GpuMatrix storage round trips
// (src/init.mjs:14-143, src/util/device.mjs:14-49, src/classes/*.mjs). On
// the GPU the same paths run through the real addon in validation.mjs --gpu
// (one device); the second device and cleanup(one) are only exercised here.
import { createRequire } from "module";
import { test, run, assert, assertEqual, assertRejects } from "./harness.mjs";
import * as wg from "../../wgblas_amd/js/index.mjs";

const stub = createRequire(import.meta.url)(process.env.WGBLAS_HIP_ADDON)._stub;

test("init() caches by options; cleanup(one) keeps the others", async () => {
  const a = await wg.init();
  assert((await wg.init()) === a, "same options -> same device");
  assert((await wg.init({ powerPreference: "high-performance", benchmark: false })) === a,
         "the defaults resolved -> the same key");
  const b = await wg.init({ benchmark: true });
  assert(b !== a && b._ctx !== a._ctx, "other options -> another device and context");
  assertEqual(stub.live().length, 2, "two live contexts");
  assertEqual(wg.gpuName().device, "gfx950:stub", "gpuName() names the first device");
  wg.cleanup(b);
  assert(b._ctx === null && a._ctx !== null, "cleanup(b) released b only");
  assertEqual(stub.live().length, 1, "one live context");
  assert((await wg.init()) === a, "a still cached");
  const b2 = await wg.init({ benchmark: true });
  assert(b2 !== b, "b's options make a new device after its cleanup");
  wg.cleanup(b2);
  wg.cleanup(b2);  // released twice: a no-op
  wg.cleanup({});  // not a device: ignored
  assertEqual(stub.live().length, 1);
});

test("cleanup(first) moves gpuName()'s default to a remaining device", async () => {
  const a = await wg.init();
  const b = await wg.init({ benchmark: true });
  wg.cleanup(a);
  assertEqual(wg.gpuName().device, "gfx950:stub", "gpuName() names the remaining device");
  assert(b._ctx !== null);
  wg.cleanup();
  assertEqual(stub.live().length, 0, "cleanup() released every device");
  let threw = false;
  try {
    wg.gpuName();
  } catch (e) {
    threw = /init\(\)/.test(e.message);
  }
  assert(threw, "gpuName() with no device");
});

test("operands of another device are rejected; a released device rejects calls", async () => {
  const a = await wg.init();
  const b = await wg.init({ benchmark: true });
  const x = wg.GpuVector.from(b, new Float32Array([3, 4]));
  await assertRejects(() => wg.snrm2(a, 2, x, 1), "different GPUDevice", "x on b, called on a");
  const M = wg.GpuMatrix.from(a, new Float32Array([1, 2, 99, 3, 4, 99]), 2, 2, 3);
  const back = await M.read();
  assertEqual(back.length, 4);
  assert(back[0] === 1 && back[1] === 2 && back[2] === 3 && back[3] === 4, "lda padding stripped");
  const v = await x.read();
  assert(v[0] === 3 && v[1] === 4, "GpuVector round trip");
  wg.cleanup(b);
  x.destroy();  // its device is gone: a no-op
  await assertRejects(() => wg.snrm2(b, 2, new Float32Array([3, 4]), 1), "released by cleanup", "call on b");
  M.destroy();
  wg.cleanup();
});

run();
