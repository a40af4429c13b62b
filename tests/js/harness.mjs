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
  const failures = [];
  for (const c of cases) {
    try {
      await c.fn();
      console.log(`ok   ${c.name}`);
    } catch (e) {
      failures.push(`${c.name}: ${(e && e.message) || e}`);
      console.log(`FAIL ${c.name}\n     ${(e && e.stack) || e}`);
    }
  }
  // failures again at the end, where a truncated log still shows them
  for (const f of failures) console.log(`FAILED ${f}`);
  console.log(`${cases.length - failures.length} passed, ${failures.length} failed`);
  process.exitCode = failures.length ? 1 : 0;
}
