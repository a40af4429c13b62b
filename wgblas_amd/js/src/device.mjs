// Operand guards shared by every routine (wgblas src/util/device.mjs:14-49).
import { HipDevice } from "./init.mjs";
import { GpuVector } from "./classes/GpuVector.mjs";
import { GpuMatrix } from "./classes/GpuMatrix.mjs";

/** Throws unless `device` is a handle from init(). The message keeps
 * wgblas's wording, which callers match on. */
export function requireGpuDevice(device) {
  if (!(device instanceof HipDevice)) throw new Error("device must be a GPUDevice (a HipDevice from init()).");
}

/** Throws if a GpuVector/GpuMatrix operand lives on another device. */
export function requireSameDevice(device, routine, operands) {
  for (const name of Object.keys(operands)) {
    const value = operands[name];
    if (!(value instanceof GpuVector) && !(value instanceof GpuMatrix)) continue;
    if (value.device !== device)
      throw new Error(
        `${routine}: ${name} belongs to a different GPUDevice than the one passed in. ` +
          "Device buffers cannot be shared across devices — recreate the operand on this " +
          "device, or call the routine with the device that owns it.",
      );
  }
}
