// TypeScript declarations for the seeded-input helpers (src/random.mjs).

/**
 * n values uniform in [low, high) (defaults -1, 1). With `seed`, the values
 * are a mulberry32 stream (the same bits for the same seed); without, Math.random.
 */
export declare function randomFloat32Array(n: number, low?: number, high?: number, seed?: number): Float32Array;
/** The same as randomFloat32Array, stored as doubles. */
export declare function randomFloat64Array(n: number, low?: number, high?: number, seed?: number): Float64Array;
/**
 * An n x n triangular matrix in an n*lda array: the `uplo` triangle's
 * off-diagonal entries uniform in [low, high) (defaults -1, 1), the diagonal
 * in [diagLow, diagHigh) (defaults 5, 15), every other entry 0; throws if
 * lda < n.
 */
export declare function randomTriangularFloat32Array(
  n: number,
  lda: number,
  uplo?: "lower" | "upper",
  low?: number,
  high?: number,
  diagLow?: number,
  diagHigh?: number,
  layout?: "row-major" | "column-major",
): Float32Array;
