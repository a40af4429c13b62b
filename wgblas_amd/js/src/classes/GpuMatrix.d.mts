// TypeScript declarations for GpuMatrix (src/classes/GpuMatrix.mjs).
import { HipDevice } from "../init.mjs";

type Data = Float32Array | Float64Array;
type Layout = "row-major" | "column-major";

/**
 * A matrix held in device memory (HBM). `rows` / `cols` are the logical
 * shape in either layout; `lda` is the stride between rows (row-major) or
 * columns (column-major); the allocation holds outer*lda elements of
 * `dtype` (Float64Array data is kept as native doubles).
 */
export declare class GpuMatrix {
  private constructor();
  readonly rows: number;
  readonly cols: number;
  readonly lda: number;
  readonly layout: Layout;
  readonly dtype: Float32ArrayConstructor | Float64ArrayConstructor;
  readonly device: HipDevice;

  /** Uploads `data` (at least outer*lda elements) to the device from the first `init()`. */
  static from(data: Data, rows: number, cols: number, lda?: number, layout?: Layout): GpuMatrix;
  /** Uploads `data` to `device`; the matrix belongs to that device for life. */
  static from(device: HipDevice, data: Data, rows: number, cols: number, lda?: number, layout?: Layout): GpuMatrix;

  /** Copies the matrix back, dense (lda padding dropped), in its layout. */
  read(): Promise<Float32Array | Float64Array>;
  /** Frees the device allocation; safe to call twice. */
  destroy(): void;
}
