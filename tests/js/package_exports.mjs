// The package surface (wgblas_amd/js/package.json) against wgblas's
// (package.json:7-33 and the per-routine entries after it): every subpath
// resolves to a module that loads without a GPU, carries a `types`
// condition whose declaration file exists, and that file declares every
// name the module exports at run time (functions, classes, re-exports).
import { readFileSync, existsSync } from "fs";
import { fileURLToPath, pathToFileURL } from "url";
import { dirname, join } from "path";
import { test, run, assert } from "./harness.mjs";

const here = dirname(fileURLToPath(import.meta.url));
const pkgDir = join(here, "..", "..", "wgblas_amd", "js");
const pkg = JSON.parse(readFileSync(join(pkgDir, "package.json"), "utf8"));

// Names a declaration file provides: declared functions / classes / types
// and the names of `export { a, b } from` re-exports.
function declaredNames(path) {
  const text = readFileSync(path, "utf8");
  const names = new Set();
  for (const m of text.matchAll(/export declare (?:function|class) (\w+)/g)) names.add(m[1]);
  for (const m of text.matchAll(/export (?:type )?\{([^}]*)\} from/g))
    for (const n of m[1].split(",")) if (n.trim()) names.add(n.trim().split(/\s+as\s+/).pop());
  return names;
}

test("package.json names index.d.mts as the root types", () => {
  assert(pkg.types === "./index.d.mts", `types = ${pkg.types}`);
  assert(existsSync(join(pkgDir, pkg.types)), "index.d.mts exists");
});

test("wgblas's public subpaths for this path are all exported", () => {
  const want = ["./random", "./classes/GpuVector", "./classes/GpuMatrix", "./sgemm", "./sgemmtr", "./ssyrk",
    "./dgemm", "./dgemmtr", "./dsyrk", "./ssyr2k", "./ssymm", "./strmm", "./strsm", "./dsyr2k", "./dsymm",
    "./dtrmm", "./sgemv", "./sdot", "./sasum", "./snrm2", "./isamax", "./ddot", "./dasum", "./dnrm2", "./idamax"];
  for (const w of want) assert(w in pkg.exports, `missing subpath ${w}`);
});

for (const [sub, target] of Object.entries(pkg.exports)) {
  test(`subpath ${sub}: import and types`, async () => {
    assert(typeof target === "object" && target.import && target.types, `${sub} needs import and types conditions`);
    const keys = Object.keys(target);
    assert(keys[0] === "types", `${sub}: "types" must come first (got ${keys.join(", ")})`);
    const mod = join(pkgDir, target.import);
    const decl = join(pkgDir, target.types);
    assert(existsSync(mod), `${sub}: ${target.import} missing`);
    assert(existsSync(decl), `${sub}: ${target.types} missing`);
    const m = await import(pathToFileURL(mod).href);
    const names = declaredNames(decl);
    const runtime = Object.keys(m);
    assert(runtime.length > 0, `${sub} exports nothing`);
    for (const n of runtime) assert(names.has(n), `${sub}: ${n} is exported but not declared in ${target.types}`);
  });
}

run();
