// A host-memory stand-in for the Node-API addon's context and memory calls
// (init / destroy / deviceName / setTiming / lastTimeMs / malloc / free /
// upload / download), loaded through WGBLAS_HIP_ADDON by devices_cpu.mjs to
// check the JS layer's device handling on the CPU. It has no compute calls:
// a routine that reaches one fails. Every call on a destroyed context throws,
// so a use after cleanup() is seen.
"use strict";

let nextId = 1;
const live = new Map();  // context id -> { buffers: Map, timing }
const destroyed = [];

function ctxOf(c) {
  if (!c || !live.has(c.id)) throw new Error("stub addon: context used after destroy");
  return live.get(c.id);
}

module.exports = {
  deviceCount: () => 1,
  init(index) {
    const c = { id: nextId++, index };
    live.set(c.id, { buffers: new Map(), timing: false, nextBuf: 1 });
    return c;
  },
  destroy(c) {
    ctxOf(c);
    live.delete(c.id);
    destroyed.push(c.id);
  },
  deviceName(c) {
    ctxOf(c);
    return { name: "stub device", arch: "gfx950:stub" };
  },
  setTiming(c, on) {
    ctxOf(c).timing = !!on;
  },
  lastTimeMs(c) {
    ctxOf(c);
    return 0.5;
  },
  malloc(c, bytes) {
    const s = ctxOf(c);
    const id = s.nextBuf++;
    s.buffers.set(id, new Uint8Array(bytes));
    return { buf: id };
  },
  free(c, b) {
    ctxOf(c).buffers.delete(b.buf);
  },
  upload(c, b, arr) {
    ctxOf(c).buffers.get(b.buf).set(new Uint8Array(arr.buffer, arr.byteOffset, arr.byteLength));
  },
  download(c, b, arr) {
    const src = ctxOf(c).buffers.get(b.buf);
    new Uint8Array(arr.buffer, arr.byteOffset, arr.byteLength).set(src.subarray(0, arr.byteLength));
  },
  // for the tests: which contexts are alive / were destroyed, and a
  // buffer's bytes (cpu_addon.cjs computes on them)
  _stub: {
    live: () => [...live.keys()],
    destroyed: () => destroyed.slice(),
    bytes: (c, b) => ctxOf(c).buffers.get(b.buf),
  },
};
