// TypeScript declarations for GpuVector (src/classes/GpuVector.mjs).
import { HipDevice } from "../init.mjs";

/** A vector held in device memory (HBM), of `length` elements of `dtype`. */
export declare class GpuVector {
  private constructor();
  readonly length: number;
  readonly dtype: Float32ArrayConstructor | Float64ArrayConstructor;
  readonly device: HipDevice;

  /** Uploads `data` to the device from the first `init()`. */
  static from(data: Float32Array | Float64Array): GpuVector;
  /** Uploads `data` to `device`; the vector belongs to that device for life. */
  static from(device: HipDevice, data: Float32Array | Float64Array): GpuVector;

  /** Copies the vector back into a new array of its dtype. */
  read(): Promise<Float32Array | Float64Array>;
  /** Frees the device allocation; safe to call twice. */
  destroy(): void;
}
