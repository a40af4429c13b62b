// Seeded inputs with wgblas's contract (src/random/random.mjs:14-26): with a
// seed, element i is low + next()*(high - low) of a mulberry32 stream, in
// double precision, stored into the array's element type; without one,
// Math.random. mulberry32 is Tommy Ettinger's 32-bit generator: the state
// advances by 0x6D2B79F5 and each draw is a xorshift-multiply hash of it.

function mulberry32(seed) {
  let state = seed >>> 0;
  return function next() {
    state = (state + 0x6d2b79f5) >>> 0;
    let t = Math.imul(state ^ (state >>> 15), state | 1) >>> 0;
    t = ((t + Math.imul(t ^ (t >>> 7), t | 61)) ^ t) >>> 0;
    return ((t ^ (t >>> 14)) >>> 0) / 4294967296;
  };
}

function fill(out, low, high, seed) {
  const next = seed === undefined ? Math.random : mulberry32(seed);
  const range = high - low;
  for (let i = 0; i < out.length; i++) out[i] = low + next() * range;
  return out;
}

export function randomFloat32Array(n, low = -1, high = 1, seed) {
  return fill(new Float32Array(n), low, high, seed);
}

export function randomFloat64Array(n, low = -1, high = 1, seed) {
  return fill(new Float64Array(n), low, high, seed);
}
