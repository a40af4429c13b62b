// Device-resident matrix (wgblas src/classes/GpuMatrix.mjs). `rows`/`cols`
// are the logical shape; `lda` is the stride between rows (row-major) or
// columns (column-major); the allocation holds outer*lda elements, where
// outer is rows (row-major) or cols (column-major). The routines read
// GpuMatrix operands in place and write GpuMatrix C in place.
import { HipDevice, getDevice } from "../init.mjs";
import { native } from "../native.mjs";

export class GpuMatrix {
  constructor(buffer, rows, cols, lda, loBuffer = null, layout = "row-major", device = null,
              dtype = Float32Array) {
    this._buf = buffer;
    this._loBuf = loBuffer;
    this.rows = rows;
    this.cols = cols;
    this.lda = lda;
    this.layout = layout;
    this.dtype = dtype;
    this.device = device === null ? getDevice() : device;
  }

  /**
   * GpuMatrix.from([device,] data, rows, cols, lda?, layout = 'row-major').
   * lda defaults to cols (row-major) or rows (column-major); data must hold
   * at least outer*lda elements. Argument checks and their messages follow
   * wgblas's (src/classes/GpuMatrix.mjs:43-79).
   */
  static from(deviceOrData, ...rest) {
    const explicit = deviceOrData instanceof HipDevice;
    const device = explicit ? deviceOrData : getDevice();
    const data = explicit ? rest.shift() : deviceOrData;
    let rows = rest[0];
    let cols = rest[1];
    let lda = rest[2];
    const layout = rest[3] === undefined ? "row-major" : rest[3];
    if (layout !== "row-major" && layout !== "column-major")
      throw new Error("layout must be 'row-major' or 'column-major'.");
    const rowMajor = layout === "row-major";
    if (lda === undefined) lda = rowMajor ? cols : rows;
    if (!(data instanceof Float32Array) && !(data instanceof Float64Array))
      throw new Error(
        "GpuMatrix.from expects a Float32Array or Float64Array (complex storage is not part of this build).",
      );
    if (!Number.isInteger(rows) || rows <= 0) throw new Error("rows must be a positive integer.");
    if (!Number.isInteger(cols) || cols <= 0) throw new Error("cols must be a positive integer.");
    const minLda = rowMajor ? cols : rows;
    if (!Number.isInteger(lda) || lda < minLda)
      throw new Error(`lda must be an integer >= ${rowMajor ? "cols" : "rows"}.`);
    const outer = rowMajor ? rows : cols;
    if (data.length < outer * lda)
      throw new Error("data does not have enough elements for the given rows, cols, and lda.");
    const view = data.subarray(0, outer * lda);
    const nat = native();
    const ctx = device.ctx();
    const buf = nat.malloc(ctx, view.byteLength);
    try {
      nat.upload(ctx, buf, view);
    } catch (e) {
      nat.free(ctx, buf);
      throw e;
    }
    return new GpuMatrix(buf, rows, cols, lda, null, layout, device, data.constructor);
  }

  /** Copies the matrix back, dense (lda padding stripped), in its layout. */
  async read() {
    const rowMajor = this.layout !== "column-major";
    const outer = rowMajor ? this.rows : this.cols;
    const inner = rowMajor ? this.cols : this.rows;
    const raw = new this.dtype(outer * this.lda);
    native().download(this.device.ctx(), this._buf, raw);
    if (this.lda === inner) return raw;
    const out = new this.dtype(outer * inner);
    for (let r = 0; r < outer; r++) out.set(raw.subarray(r * this.lda, r * this.lda + inner), r * inner);
    return out;
  }

  /** Frees the device allocation (safe to call twice). */
  destroy() {
    if (this._buf !== null && this.device._ctx !== null) native().free(this.device._ctx, this._buf);
    this._buf = null;
  }
}
