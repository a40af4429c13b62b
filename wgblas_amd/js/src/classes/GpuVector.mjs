// Device-resident vector (wgblas src/classes/GpuVector.mjs): an HBM
// allocation the routines read in place. from() uploads, read() copies back,
// destroy() frees. Float64Array data is kept as native doubles (wgblas splits
// it into a double-double hi/lo pair; here `_loBuf` is always null).
import { HipDevice, getDevice } from "../init.mjs";
import { native } from "../native.mjs";

export class GpuVector {
  constructor(buffer, length, dtype = Float32Array, loBuffer = null, device = null) {
    this._buf = buffer;
    this._loBuf = loBuffer;
    this.length = length;
    this.dtype = dtype;
    this.device = device === null ? getDevice() : device;
  }

  /** GpuVector.from([device,] data): uploads a Float32Array or Float64Array. */
  static from(deviceOrData, maybeData) {
    const explicit = deviceOrData instanceof HipDevice;
    const device = explicit ? deviceOrData : getDevice();
    const data = explicit ? maybeData : deviceOrData;
    if (!(data instanceof Float32Array) && !(data instanceof Float64Array))
      throw new Error(
        "GpuVector.from expects a Float32Array or Float64Array (complex storage is not part of this build).",
      );
    const nat = native();
    const ctx = device.ctx();
    const buf = nat.malloc(ctx, data.byteLength);
    try {
      nat.upload(ctx, buf, data);
    } catch (e) {
      nat.free(ctx, buf);
      throw e;
    }
    return new GpuVector(buf, data.length, data.constructor, null, device);
  }

  /** Copies the vector back into a new typed array of its dtype. */
  async read() {
    const out = new this.dtype(this.length);
    if (this.length > 0) native().download(this.device.ctx(), this._buf, out);
    return out;
  }

  /** Frees the device allocation (safe to call twice). */
  destroy() {
    if (this._buf !== null && this.device._ctx !== null) native().free(this.device._ctx, this._buf);
    this._buf = null;
  }
}
