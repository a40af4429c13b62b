// Minimal test runner for the JavaScript layer (Node 12 has no node:test):
// test(name, fn) queues a case, run() executes them in order and exits
// non-zero when any failed. Used by tests/test_js_*.py through `node`.
const cases = [];

export function test(name, fn) {
  cases.push({ name, fn });
}

export class AssertionError extends Error {}

export function assert(cond, msg) {
  if (!cond) throw new AssertionError(msg || "assertion failed");
}

export function assertEqual(got, want, msg) {
  if (!Object.is(got, want) && !(got === want))
    throw new AssertionError(`${msg || "not equal"}: got ${got}, want ${want}`);
}

export async function assertRejects(fn, substring, msg) {
  let threw = false;
  try {
    await fn();
  } catch (e) {
    threw = true;
    if (!String(e && e.message).includes(substring))
      throw new AssertionError(`${msg || "wrong error"}: expected "${substring}", got "${e && e.message}"`);
  }
  if (!threw) throw new AssertionError(`${msg || "did not throw"}: expected "${substring}"`);
}

export async function run() {
  let failed = 0;
  for (const c of cases) {
    try {
      await c.fn();
      console.log(`ok   ${c.name}`);
    } catch (e) {
      failed++;
      console.log(`FAIL ${c.name}\n     ${(e && e.stack) || e}`);
    }
  }
  console.log(`${cases.length - failed} passed, ${failed} failed`);
  process.exitCode = failed ? 1 : 0;
}
