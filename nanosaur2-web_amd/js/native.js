// Loads the ns2 N-API addon (lib/ns2.node, built by `make -C nanosaur2-web_amd`). There is no
// fallback: without the addon every op would be unavailable, so loading fails loudly.
import { createRequire } from "module";
import { fileURLToPath } from "url";
import { existsSync } from "fs";

const require = createRequire(import.meta.url);
const addonPath = fileURLToPath(new URL("../lib/ns2.node", import.meta.url));
if (!existsSync(addonPath)) {
  throw new Error(`ns2 addon not built: ${addonPath} is missing (run make -C nanosaur2-web_amd)`);
}

export const native = require(addonPath);
export const ACT = { none: 0, silu: 1, gelu_tanh: 2 };
export const EW = { add: 0, sub: 1, silu: 2, copy: 3 };
