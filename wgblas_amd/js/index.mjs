// wgblas's public API for the hot path, on HIP (the routine set of
// index.mjs in wgblas limited to the GEMM family, the level-3 routines built
// on it and the level-1 reductions, plus the device, residency and
// seeded-input helpers).
export { init, cleanup, gpuName, HipDevice } from "./src/init.mjs";
export { GpuVector } from "./src/classes/GpuVector.mjs";
export { GpuMatrix } from "./src/classes/GpuMatrix.mjs";
export { randomFloat32Array, randomFloat64Array, randomTriangularFloat32Array } from "./src/random.mjs";
export { sgemm } from "./src/sgemm.mjs";
export { sgemmtr } from "./src/sgemmtr.mjs";
export { ssyrk } from "./src/ssyrk.mjs";
export { dgemm } from "./src/dgemm.mjs";
export { dgemmtr } from "./src/dgemmtr.mjs";
export { dsyrk } from "./src/dsyrk.mjs";
export { ssyr2k } from "./src/ssyr2k.mjs";
export { ssymm } from "./src/ssymm.mjs";
export { strmm } from "./src/strmm.mjs";
export { dsyr2k } from "./src/dsyr2k.mjs";
export { dsymm } from "./src/dsymm.mjs";
export { dtrmm } from "./src/dtrmm.mjs";
export { strsm } from "./src/strsm.mjs";
export { sgemv } from "./src/sgemv.mjs";
export { dgemv } from "./src/dgemv.mjs";
export { sger } from "./src/sger.mjs";
export { dger } from "./src/dger.mjs";
export { ssyr } from "./src/ssyr.mjs";
export { dsyr } from "./src/dsyr.mjs";
export { ssyr2 } from "./src/ssyr2.mjs";
export { dsyr2 } from "./src/dsyr2.mjs";
export { ssymv } from "./src/ssymv.mjs";
export { dsymv } from "./src/dsymv.mjs";
export { strmv } from "./src/strmv.mjs";
export { dtrmv } from "./src/dtrmv.mjs";
export { sdot } from "./src/sdot.mjs";
export { sasum } from "./src/sasum.mjs";
export { snrm2 } from "./src/snrm2.mjs";
export { isamax } from "./src/isamax.mjs";
export { ddot } from "./src/ddot.mjs";
export { dasum } from "./src/dasum.mjs";
export { dnrm2 } from "./src/dnrm2.mjs";
export { idamax } from "./src/idamax.mjs";
