// Loads the Node-API addon (wgblas_amd/lib/wgblas_hip.node), which binds
// libwgblas_hip's C ABI. There is no fallback: without the addon every
// routine fails with the error below.
import { createRequire } from "module";
import { fileURLToPath } from "url";
import { dirname, join } from "path";

const here = dirname(fileURLToPath(import.meta.url));
const addonPath = process.env.WGBLAS_HIP_ADDON || join(here, "..", "..", "lib", "wgblas_hip.node");

let addon = null;
let loadError = null;
try {
  addon = createRequire(import.meta.url)(addonPath);
} catch (e) {
  loadError = e;
}

/** The addon's functions; throws if the addon could not be loaded. */
export function native() {
  if (addon === null)
    throw new Error(
      `wgblas HIP addon not available (${addonPath}): build it with ` +
        "`python -m wgblas_amd.build` — " + (loadError ? loadError.message : "unknown error"),
    );
  return addon;
}
