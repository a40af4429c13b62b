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

/**
 * An n x n triangular matrix in an n*lda array for the triangular routines'
 * examples and tests (wgblas src/random/random.mjs:28-60): the `uplo`
 * triangle's off-diagonal entries uniform in [low, high), the diagonal in
 * [diagLow, diagHigh) (away from zero, so a solve has no tiny pivot), every
 * other entry 0. `uplo` names the logical triangle in either storage order;
 * entry (i, j) sits at i*lda + j (row-major) or j*lda + i (column-major).
 * Draws come from Math.random, row by row (row-major) or column by column.
 */
export function randomTriangularFloat32Array(n, lda, uplo = "lower", low = -1, high = 1, diagLow = 5,
                                             diagHigh = 15, layout = "row-major") {
  if (uplo !== "lower" && uplo !== "upper") throw new Error("uplo must be 'lower' or 'upper'.");
  if (layout !== "row-major" && layout !== "column-major")
    throw new Error("layout must be 'row-major' or 'column-major'.");
  if (lda < n) throw new Error("lda must be >= n.");
  const out = new Float32Array(n * lda);
  // Walk the storage order's outer index; the triangle of outer line o is
  // the inner indices below (lower row-major / upper column-major) or above
  // it, the diagonal last.
  const leading = (uplo === "lower") === (layout === "row-major");
  for (let o = 0; o < n; o++) {
    const line = o * lda;
    const [from, to] = leading ? [0, o] : [o + 1, n];
    for (let i = from; i < to; i++) out[line + i] = low + Math.random() * (high - low);
    out[line + o] = diagLow + Math.random() * (diagHigh - diagLow);
  }
  return out;
}
