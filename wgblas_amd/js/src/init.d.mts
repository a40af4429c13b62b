// TypeScript declarations for device bring-up (src/init.mjs).

/**
 * The handle `init()` returns and every routine takes first: one HIP device
 * and one stream on which the routines' work is ordered.
 */
export declare class HipDevice {
  private constructor();
  /** HIP device index (WGBLAS_HIP_DEVICE, default 0). */
  readonly index: number;
  /** The resolved options this device was created with. */
  readonly options: { powerPreference: string; benchmark: boolean; dumpShaders: boolean };
  /** True when created with `benchmark: true`: routines also return `gpuTimeMs`. */
  readonly benchmark: boolean;
}

/**
 * Opens the device, or returns the cached one for the same options.
 * `benchmark: true` adds `gpuTimeMs` (HIP events around the call's kernels)
 * to every routine's result. `powerPreference` only keys the cache and
 * `dumpShaders` only warns: the kernels are precompiled for gfx950.
 */
export declare function init(options?: {
  powerPreference?: "high-performance" | "low-power";
  benchmark?: boolean;
  dumpShaders?: boolean;
}): Promise<HipDevice>;

/** Releases one device, or every device when called without one; unknown or released devices are ignored. */
export declare function cleanup(device?: HipDevice): void;

/** Marketing name and gfx architecture of a device (default: the first one `init()` opened). */
export declare function gpuName(device?: HipDevice): { description: string; device: string };
