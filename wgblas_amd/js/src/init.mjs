// Device bring-up: wgblas's init / cleanup / gpuName (src/init.mjs:31-143)
// on HIP. A HipDevice stands where wgblas hands out a GPUDevice: it owns one
// libwgblas_hip context (one HIP device, one stream) and is passed as the
// first argument of every routine.
import { native } from "./native.mjs";

/** Handle returned by init(); the `device` argument of every routine. */
export class HipDevice {
  constructor(ctx, index, options) {
    this._ctx = ctx; // napi external wrapping the wgb_ctx; null once released
    this.index = index;
    this.options = options;
    this.benchmark = !!options.benchmark;
    this.lost = false;
  }

  /** The live context, or an error if cleanup() already released it. */
  ctx() {
    if (this._ctx === null) throw new Error("This device was released by cleanup().");
    return this._ctx;
  }
}

// Options key -> HipDevice: init() with the same options returns the same
// device, and each distinct option set gets its own context (as wgblas keys
// its GPUDevices by powerPreference and benchmark).
const devices = new Map();
let primary = null;
let warnedShaders = false;

const optionsKey = (o) => `${o.powerPreference}::${o.benchmark}`;

/**
 * Opens the HIP device and returns its handle. `powerPreference` only keys
 * the cache (every MI355X is a discrete device); the device index comes from
 * WGBLAS_HIP_DEVICE (default 0). `benchmark: true` makes every routine also
 * return `gpuTimeMs`, measured with HIP events around its kernels.
 * `dumpShaders` has no meaning without a shader compiler and only warns.
 */
export async function init(options) {
  const o = options || {};
  const resolved = {
    powerPreference: o.powerPreference === undefined ? "high-performance" : o.powerPreference,
    benchmark: o.benchmark === undefined ? false : o.benchmark,
    dumpShaders: o.dumpShaders === undefined ? false : o.dumpShaders,
  };
  const key = optionsKey(resolved);
  const cached = devices.get(key);
  if (cached) return cached;
  if (resolved.dumpShaders && !warnedShaders) {
    warnedShaders = true;
    console.warn("dumpShaders has no effect on the HIP backend (the kernels are precompiled for gfx950).");
  }
  const nat = native();
  if (nat.deviceCount() < 1) throw new Error("No HIP device found.");
  const index = process.env.WGBLAS_HIP_DEVICE ? Number(process.env.WGBLAS_HIP_DEVICE) : 0;
  const ctx = nat.init(index);
  const device = new HipDevice(ctx, index, resolved);
  if (device.benchmark) nat.setTiming(ctx, true);
  devices.set(key, device);
  if (!primary) primary = device;
  return device;
}

/** Releases one device, or every device when called without one. Unknown or
 * already-released devices are ignored. */
export function cleanup(device) {
  const nat = native();
  if (device === undefined) {
    for (const d of devices.values()) {
      if (d._ctx !== null) nat.destroy(d._ctx);
      d._ctx = null;
    }
    devices.clear();
    primary = null;
    return;
  }
  if (!(device instanceof HipDevice) || device._ctx === null) return;
  devices.delete(optionsKey(device.options));
  nat.destroy(device._ctx);
  device._ctx = null;
  if (primary === device) {
    const next = devices.values().next();
    primary = next.done ? null : next.value;
  }
}

/** { description: marketing name, device: gfx architecture } of a device
 * (default: the first one init() created). */
export function gpuName(device) {
  const d = device === undefined ? primary : device;
  if (!(d instanceof HipDevice) || d._ctx === null)
    throw new Error("HIP device not initialized — call init() first.");
  const info = native().deviceName(d._ctx);
  return { description: info.name || "unknown", device: info.arch || "unknown" };
}

/** The device from the first init(); GpuVector.from(data) and
 * GpuMatrix.from(data, ...) use it when no device is passed. */
export function getDevice() {
  if (!primary) throw new Error("HIP device not initialized — call init() first.");
  return primary;
}

/** gpuTimeMs of the call just made on `device` when benchmark mode is on. */
export function lastGpuTimeMs(device) {
  if (!device.benchmark) return undefined;
  return native().lastTimeMs(device.ctx());
}
