// A host-memory stand-in for the whole Node-API addon (wgblas_hip.node):
// stub_addon.cjs's context and memory calls plus every compute call, done
// on the CPU in float64 (fp32 routines round each result to float32 once),
// with the C ABI's own semantics (include/wgblas_hip.h): column-major
// operands, the quick returns, the alpha / beta read rules and reference
// BLAS's zero skipping where the library keeps it. Loaded through
// WGBLAS_HIP_ADDON, it lets the JS layer's routines (argument checks, layout
// and uplo mapping, residency, narrowing, result shapes) run their GPU
// suites end to end without a GPU; the kernels themselves are checked on
// the GPU through the C ABI by the pytest suites.
"use strict";

const stub = require("./stub_addon.cjs");

// CPU_ADDON_PLANT: one deliberate mistake, for the test that shows the
// suites fail on it: "trans" (gemm reads op(A) as A), "uplo" (gemm / ssyrk
// on a triangle write the whole of C), "amax" (isamax keeps the last of
// equal magnitudes)
const PLANT = process.env.CPU_ADDON_PLANT || "";

const f32 = (c, b) => {
  const u8 = stub._stub.bytes(c, b);
  return new Float32Array(u8.buffer, u8.byteOffset, u8.byteLength >> 2);
};
const f64 = (c, b) => {
  const u8 = stub._stub.bytes(c, b);
  return new Float64Array(u8.buffer, u8.byteOffset, u8.byteLength >> 3);
};
const view = (c, b, dbl) => (dbl ? f64(c, b) : f32(c, b));
const rnd = (dbl) => (dbl ? (v) => v : Math.fround);
const LOWER = 1;
const LEFT = 1;

function gemmCore(dbl, uplo, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc) {
  const r = rnd(dbl);
  if (!dbl) {
    alpha = Math.fround(alpha);
    beta = Math.fround(beta);
  }
  if (m === 0 || n === 0) return;
  if (dbl && (alpha === 0 || k === 0) && beta === 1) return;  // C untouched
  for (let j = 0; j < n; ++j)
    for (let i = 0; i < m; ++i) {
      if (PLANT !== "uplo" && (uplo === 1 ? i < j : uplo === 2 ? i > j : false)) continue;
      let s = 0;
      const tA = PLANT === "trans" ? 0 : ta;
      if (alpha !== 0)
        for (let p = 0; p < k; ++p)
          s += (tA ? A[p + i * lda] : A[i + p * lda]) * (tb ? B[j + p * ldb] : B[p + j * ldb]);
      let v = alpha === 0 ? 0 : alpha * s;
      if (beta !== 0) v += beta * C[i + j * ldc];
      C[i + j * ldc] = r(v);
    }
}

// sum / abs-sum / norm / first index of the largest magnitude, with the
// library's rules (norm scaled to stay in range; index: NaN never wins, an
// all-NaN vector gives 0)
function reduceCore(kind, n, x, incx, y, incy) {
  const dbl = kind >= 4, r = rnd(dbl), op = kind % 4;
  if (op === 0) {
    let s = 0;
    for (let i = 0; i < n; ++i) s += x[i * incx] * y[i * incy];
    return r(s);
  }
  if (op === 1) {
    let s = 0;
    for (let i = 0; i < n; ++i) s += Math.abs(x[i * incx]);
    return r(s);
  }
  if (op === 2) {
    let amax = 0, nan = false;
    for (let i = 0; i < n; ++i) {
      const a = Math.abs(x[i * incx]);
      if (Number.isNaN(a)) nan = true;
      else if (a > amax) amax = a;
    }
    if (nan) return NaN;
    if (amax === 0 || amax === Infinity) return amax;
    let s = 0;
    for (let i = 0; i < n; ++i) {
      const t = x[i * incx] / amax;
      s += t * t;
    }
    return r(amax * Math.sqrt(s));
  }
  let best = -1, at = 0;
  for (let i = 0; i < n; ++i) {
    const a = Math.abs(x[i * incx]);
    if (PLANT === "amax" ? a >= best : a > best) {
      best = a;
      at = i;
    }
  }
  return at;
}

const compute = {
  // gemm(kind, ctx, uplo, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc):
  // 0 sgemm, 1 sgemmtr, 2 dgemm, 3 dgemmtr
  gemm(kind, c, uplo, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc) {
    const dbl = kind >= 2;
    gemmCore(dbl, kind % 2 ? uplo : 0, ta, tb, m, n, k, alpha, view(c, A, dbl), lda, view(c, B, dbl), ldb,
             beta, view(c, C, dbl), ldc);
  },
  // ssyrk(ctx, uplo, trans, n, k, alpha, A, lda, beta, C, ldc[, f64])
  ssyrk(c, uplo, trans, n, k, alpha, A, lda, beta, C, ldc, dbl) {
    const a = view(c, A, !!dbl);
    gemmCore(!!dbl, uplo, trans, trans ? 0 : 1, n, n, k, alpha, a, lda, a, lda, beta, view(c, C, !!dbl), ldc);
  },
  // ssyr2k(ctx, uplo, transA, transB, n, k, alpha, A, lda, B, ldb, beta, C, ldc[, f64])
  ssyr2k(c, uplo, ta, tb, n, k, alpha, A, lda, B, ldb, beta, C, ldc, dbl) {
    dbl = !!dbl;
    const r = rnd(dbl), a = view(c, A, dbl), b = view(c, B, dbl), cm = view(c, C, dbl);
    if (!dbl) {
      alpha = Math.fround(alpha);
      beta = Math.fround(beta);
    }
    if (n === 0 || (dbl && (alpha === 0 || k === 0) && beta === 1)) return;
    const opA = (i, p) => (ta ? a[p + i * lda] : a[i + p * lda]);
    const opB = (i, p) => (tb ? b[p + i * ldb] : b[i + p * ldb]);
    for (let j = 0; j < n; ++j)
      for (let i = 0; i < n; ++i) {
        if (uplo === LOWER ? i < j : i > j) continue;
        let s = 0;
        if (alpha !== 0) for (let p = 0; p < k; ++p) s += opA(i, p) * opB(j, p) + opB(i, p) * opA(j, p);
        let v = alpha === 0 ? 0 : alpha * s;
        if (beta !== 0) v += beta * cm[i + j * ldc];
        cm[i + j * ldc] = r(v);
      }
  },
  // ssymm(ctx, side, uplo, transB, m, n, alpha, A, lda, B, ldb, beta, C, ldc[, f64])
  ssymm(c, side, uplo, tb, m, n, alpha, A, lda, B, ldb, beta, C, ldc, dbl) {
    dbl = !!dbl;
    const r = rnd(dbl), a = view(c, A, dbl), b = view(c, B, dbl), cm = view(c, C, dbl);
    if (!dbl) {
      alpha = Math.fround(alpha);
      beta = Math.fround(beta);
    }
    if (m === 0 || n === 0 || (dbl && alpha === 0 && beta === 1)) return;
    const S = (i, p) => ((uplo === LOWER ? i >= p : i <= p) ? a[i + p * lda] : a[p + i * lda]);
    const opB = (i, j) => (tb ? b[j + i * ldb] : b[i + j * ldb]);
    const order = side === LEFT ? m : n;
    for (let j = 0; j < n; ++j)
      for (let i = 0; i < m; ++i) {
        let s = 0;
        if (alpha !== 0)
          for (let p = 0; p < order; ++p) s += side === LEFT ? S(i, p) * opB(p, j) : opB(i, p) * S(p, j);
        let v = alpha === 0 ? 0 : alpha * s;
        if (beta !== 0) v += beta * cm[i + j * ldc];
        cm[i + j * ldc] = r(v);
      }
  },
  // tri(kind, ctx, side, uplo, transA, diag, m, n, alpha, A, lda, B, ldb):
  // 0 strmm, 1 strsm, 2 dtrmm
  tri(kind, c, side, uplo, trans, diag, m, n, alpha, A, lda, B, ldb) {
    const dbl = kind === 2, r = rnd(dbl), a = view(c, A, dbl), b = view(c, B, dbl);
    if (!dbl) alpha = Math.fround(alpha);
    if (m === 0 || n === 0) return;
    const opLower = (uplo === LOWER) !== (trans !== 0);
    // op(A)[i, k] over the triangle; undefined outside it
    const T = (i, k) => {
      if (i === k) return diag ? 1 : a[i + i * lda];
      if (opLower ? i < k : i > k) return undefined;
      return trans ? a[k + i * lda] : a[i + k * lda];
    };
    const order = side === LEFT ? m : n;
    if (kind !== 1) {
      const out = new Float64Array(m * n);
      for (let j = 0; j < n; ++j)
        for (let i = 0; i < m; ++i) {
          let s = 0;
          if (alpha !== 0)
            for (let p = 0; p < order; ++p) {
              const e = side === LEFT ? T(i, p) : T(p, j);
              if (e === undefined) continue;
              s += side === LEFT ? e * b[p + j * ldb] : b[i + p * ldb] * e;
            }
          out[i + j * m] = alpha === 0 ? 0 : alpha * s;
        }
      for (let j = 0; j < n; ++j) for (let i = 0; i < m; ++i) b[i + j * ldb] = r(out[i + j * m]);
      return;
    }
    const nrhs = side === LEFT ? n : m;
    const forward = side === LEFT ? opLower : !opLower;
    const at = (i, rh) => (side === LEFT ? i + rh * ldb : rh + i * ldb);
    for (let rh = 0; rh < nrhs; ++rh) {
      const x = new Float64Array(order);
      for (let q = 0; q < order; ++q) {
        const i = forward ? q : order - 1 - q;
        if (alpha === 0) {
          x[i] = 0;
          continue;
        }
        let s = alpha * b[at(i, rh)];
        for (let qq = 0; qq < q; ++qq) {
          const k = forward ? qq : order - 1 - qq;
          const e = side === LEFT ? T(i, k) : T(k, i);
          if (e === undefined) continue;
          s -= e * x[k];
        }
        x[i] = r(s / T(i, i));
      }
      for (let i = 0; i < order; ++i) b[at(i, rh)] = r(x[i]);
    }
  },
  // sgemv(ctx, trans, m, n, alpha, A, lda, x, incx, beta, y, incy[, f64])
  sgemv(c, trans, m, n, alpha, A, lda, X, incx, beta, Y, incy, dbl) {
    dbl = !!dbl;
    const r = rnd(dbl), a = view(c, A, dbl), x = view(c, X, dbl), y = view(c, Y, dbl);
    if (!dbl) {
      alpha = Math.fround(alpha);
      beta = Math.fround(beta);
    }
    if (m === 0 || n === 0 || (alpha === 0 && beta === 1)) return;
    const len = trans ? n : m, terms = trans ? m : n;
    for (let i = 0; i < len; ++i) {
      let s = 0;
      if (alpha !== 0)
        for (let p = 0; p < terms; ++p) {
          const xv = x[p * incx];
          if (!trans && xv === 0) continue;  // the skipped column
          s += (trans ? a[p + i * lda] : a[i + p * lda]) * xv;
        }
      let v = alpha === 0 ? 0 : alpha * s;
      if (beta !== 0) v += beta * y[i * incy];
      y[i * incy] = r(v);
    }
  },
  // ger(ctx, m, n, alpha, x, incx, y, incy, A, lda, f64)
  ger(c, m, n, alpha, X, incx, Y, incy, A, lda, dbl) {
    const r = rnd(dbl), x = view(c, X, dbl), y = view(c, Y, dbl), a = view(c, A, dbl);
    if (!dbl) alpha = Math.fround(alpha);
    if (m === 0 || n === 0 || alpha === 0) return;
    for (let j = 0; j < n; ++j) {
      const yj = y[j * incy];
      if (yj === 0) continue;
      const t = alpha * yj;
      for (let i = 0; i < m; ++i) a[i + j * lda] = r(a[i + j * lda] + x[i * incx] * t);
    }
  },
  // syr(ctx, uplo, n, alpha, x, incx, y | null, incy, A, lda, f64)
  syr(c, uplo, n, alpha, X, incx, Y, incy, A, lda, dbl) {
    const r = rnd(dbl), x = view(c, X, dbl), two = Y !== null && Y !== undefined;
    const y = two ? view(c, Y, dbl) : null, a = view(c, A, dbl);
    if (!dbl) alpha = Math.fround(alpha);
    if (n === 0 || alpha === 0) return;
    for (let j = 0; j < n; ++j) {
      const xj = x[j * incx], yj = two ? y[j * incy] : xj;
      if (xj === 0 && (!two || yj === 0)) continue;
      const t1 = alpha * yj, t2 = alpha * xj;
      const lo = uplo === LOWER ? j : 0, hi = uplo === LOWER ? n : j + 1;
      for (let i = lo; i < hi; ++i) {
        let v = a[i + j * lda] + x[i * incx] * t1;
        if (two) v += y[i * incy] * t2;
        a[i + j * lda] = r(v);
      }
    }
  },
  // symv(ctx, uplo, n, alpha, A, lda, x, incx, beta, y, incy, f64)
  symv(c, uplo, n, alpha, A, lda, X, incx, beta, Y, incy, dbl) {
    const r = rnd(dbl), a = view(c, A, dbl), x = view(c, X, dbl), y = view(c, Y, dbl);
    if (!dbl) {
      alpha = Math.fround(alpha);
      beta = Math.fround(beta);
    }
    if (n === 0 || (alpha === 0 && beta === 1)) return;
    const out = new Float64Array(n);
    for (let i = 0; i < n; ++i) {
      let s = 0;
      if (alpha !== 0)
        for (let j = 0; j < n; ++j) {
          const sij = (uplo === LOWER ? i >= j : i <= j) ? a[i + j * lda] : a[j + i * lda];
          s += sij * x[j * incx];
        }
      let v = alpha === 0 ? 0 : alpha * s;
      if (beta !== 0) v += beta * y[i * incy];
      out[i] = v;
    }
    for (let i = 0; i < n; ++i) y[i * incy] = r(out[i]);
  },
  // trmv(ctx, uplo, trans, diag, n, A, lda, x, incx, y, incy, f64)
  trmv(c, uplo, trans, diag, n, A, lda, X, incx, Y, incy, dbl) {
    const r = rnd(dbl), a = view(c, A, dbl), x = view(c, X, dbl), y = view(c, Y, dbl);
    for (let i = 0; i < n; ++i) {
      let s = 0;
      for (let j = 0; j < n; ++j) {
        const rr = trans ? j : i, cc = trans ? i : j;
        if (!(uplo === LOWER ? rr >= cc : rr <= cc)) continue;
        const xj = x[j * incx];
        if (!trans && xj === 0) continue;
        s += (diag && rr === cc ? 1 : a[rr + cc * lda]) * xj;
      }
      y[i * incy] = r(s);
    }
  },
  // reduce(kind, ctx, n, x, incx[, y, incy]) -> number; 0 sdot, 1 sasum,
  // 2 snrm2, 3 isamax, 4 ddot, 5 dasum, 6 dnrm2, 7 idamax
  reduce(kind, c, n, X, incx, Y, incy) {
    const dbl = kind >= 4;
    const x = view(c, X, dbl), y = kind % 4 === 0 ? view(c, Y, dbl) : null;
    return reduceCore(kind, n, x, incx, y, incy);
  },
};

module.exports = Object.assign({}, stub, compute);
