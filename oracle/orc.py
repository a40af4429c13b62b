"""ctypes wrapper of the CPU oracle (oracle/oracle.c) — TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker (or the timed CPU baseline). The product
(wgblas_amd/) never loads it.

Function provenance (reference file:line each one restates) is in oracle.c.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "lib", "liborc.so")

_i64, _f32p, _f64p = C.c_int64, C.POINTER(C.c_float), C.POINTER(C.c_double)
_SIG = {
    "orc_random_f32": (None, [_i64, C.c_double, C.c_double, C.c_uint32, _f32p]),
    "orc_random_f64": (None, [_i64, C.c_double, C.c_double, C.c_uint32, _f64p]),
    "orc_random_normal_f32": (None, [_i64, C.c_uint32, _f32p]),
    "orc_sdot_wgsl": (C.c_float, [_i64, _f32p, _i64, _f32p, _i64]),
    "orc_sasum_wgsl": (C.c_float, [_i64, _f32p, _i64]),
    "orc_snrm2_wgsl": (C.c_float, [_i64, _f32p, _i64]),
    "orc_isamax_wgsl": (_i64, [_i64, _f32p, _i64]),
    "orc_nrm_combine": (C.c_float, [C.c_float, C.c_float, C.c_float]),
    "orc_dot_ld": (C.c_double, [_i64, _f32p, _i64, _f32p, _i64, _f64p]),
    "orc_sum_abs_ld": (C.c_double, [_i64, _f32p, _i64]),
    "orc_nrm2_ld": (C.c_double, [_i64, _f32p, _i64]),
    "orc_isamax_brute": (_i64, [_i64, _f32p, _i64]),
    "orc_ddot_ld": (C.c_double, [_i64, _f64p, _i64, _f64p, _i64, _f64p]),
    "orc_dasum_ld": (C.c_double, [_i64, _f64p, _i64]),
    "orc_dnrm2_ld": (C.c_double, [_i64, _f64p, _i64]),
    "orc_idamax_brute": (_i64, [_i64, _f64p, _i64]),
    "orc_gemm_ld": (None, [C.c_int, C.c_int, C.c_int, _i64, _i64, _i64, C.c_double, _f64p, _i64,
                           _f64p, _i64, C.c_double, _f64p, _i64, _f64p, _i64, _f64p]),
    "orc_sgemm_wgsl": (None, [C.c_int, C.c_int, C.c_int, _i64, _i64, _i64, C.c_float, _f32p, _i64,
                              _f32p, _i64, C.c_float, _f32p, _i64]),
    "orc_ssyr2k_ld": (None, [C.c_int, C.c_int, _i64, _i64, C.c_double, _f64p, _i64, _f64p, _i64,
                             C.c_double, _f64p, _i64, _f64p, _f64p, _f64p]),
    "orc_ssymm_ld": (None, [C.c_int, C.c_int, _i64, _i64, C.c_double, _f64p, _i64, _f64p, _i64,
                            C.c_double, _f64p, _i64, _f64p, _f64p]),
    "orc_strmm_ld": (None, [C.c_int, C.c_int, C.c_int, C.c_int, _i64, _i64, C.c_double, _f64p,
                            _i64, _f64p, _i64, _f64p, _f64p]),
    "orc_strsm_ld": (None, [C.c_int, C.c_int, C.c_int, C.c_int, _i64, _i64, C.c_double, _f64p,
                            _i64, _f64p, _i64]),
    "orc_sgemv_ld": (None, [C.c_int, _i64, _i64, C.c_double, _f64p, _i64, _f64p, _i64, C.c_double,
                            _f64p, _i64, _f64p]),
    "orc_sger_ld": (None, [_i64, _i64, C.c_double, _f64p, _i64, _f64p, _i64, _f64p, _i64]),
    "orc_strmv_ld": (None, [C.c_int, C.c_int, C.c_int, _i64, _f64p, _i64, _f64p, _i64, _f64p, _i64, _f64p]),
    "orc_ssymv_ld": (None, [C.c_int, _i64, C.c_double, _f64p, _i64, _f64p, _i64, C.c_double, _f64p,
                            _i64, _f64p]),
    "orc_ssyr2_ld": (None, [C.c_int, _i64, C.c_double, _f64p, _i64, _f64p, _i64, C.c_int, _f64p, _i64]),
}

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        l = C.CDLL(LIB)
        for name, (res, args) in _SIG.items():
            fn = getattr(l, name)
            fn.restype, fn.argtypes = res, args
        _lib = l
    return _lib


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(_f32p)


def _f64(a):
    a = np.ascontiguousarray(a, dtype=np.float64)
    return a, a.ctypes.data_as(_f64p)


# ---- seeded inputs ----
def random_f32(n, low=-1.0, high=1.0, seed=0):
    out = np.empty(n, np.float32)
    lib().orc_random_f32(n, low, high, seed & 0xffffffff, out.ctypes.data_as(_f32p))
    return out


def random_f64(n, low=-1.0, high=1.0, seed=0):
    out = np.empty(n, np.float64)
    lib().orc_random_f64(n, low, high, seed & 0xffffffff, out.ctypes.data_as(_f64p))
    return out


def random_normal_f32(n, seed=0):
    out = np.empty(n, np.float32)
    lib().orc_random_normal_f32(n, seed & 0xffffffff, out.ctypes.data_as(_f32p))
    return out


# ---- level 1 ----
def sdot_wgsl(n, x, incx, y, incy):
    x, xp = _f32(x)
    y, yp = _f32(y)
    return np.float32(lib().orc_sdot_wgsl(n, xp, incx, yp, incy))


def sasum_wgsl(n, x, incx):
    x, xp = _f32(x)
    return np.float32(lib().orc_sasum_wgsl(n, xp, incx))


def snrm2_wgsl(n, x, incx):
    x, xp = _f32(x)
    return np.float32(lib().orc_snrm2_wgsl(n, xp, incx))


def isamax_wgsl(n, x, incx):
    x, xp = _f32(x)
    return int(lib().orc_isamax_wgsl(n, xp, incx))


def nrm_combine(abig, amed, asml):
    return np.float32(lib().orc_nrm_combine(abig, amed, asml))


def dot_ld(n, x, incx, y, incy):
    """(sum x*y, sum |x*y|) in long double."""
    x, xp = _f32(x)
    y, yp = _f32(y)
    a = C.c_double(0)
    s = lib().orc_dot_ld(n, xp, incx, yp, incy, C.byref(a))
    return s, a.value


def sum_abs_ld(n, x, incx):
    x, xp = _f32(x)
    return lib().orc_sum_abs_ld(n, xp, incx)


def nrm2_ld(n, x, incx):
    x, xp = _f32(x)
    return lib().orc_nrm2_ld(n, xp, incx)


def isamax_brute(n, x, incx):
    x, xp = _f32(x)
    return int(lib().orc_isamax_brute(n, xp, incx))


def ddot_ld(n, x, incx, y, incy):
    """(sum x*y, sum |x*y|) of float64 vectors in long double."""
    x, xp = _f64(x)
    y, yp = _f64(y)
    a = C.c_double(0)
    s = lib().orc_ddot_ld(n, xp, incx, yp, incy, C.byref(a))
    return s, a.value


def dasum_ld(n, x, incx):
    x, xp = _f64(x)
    return lib().orc_dasum_ld(n, xp, incx)


def dnrm2_ld(n, x, incx):
    x, xp = _f64(x)
    return lib().orc_dnrm2_ld(n, xp, incx)


def idamax_brute(n, x, incx):
    x, xp = _f64(x)
    return int(lib().orc_idamax_brute(n, xp, incx))


# ---- level 3 (column-major flat arrays) ----
def gemm_ld(uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, Cin, ldc):
    """Returns (out, absdot) as (ldc*n)-long column-major float64 arrays:
    out holds alpha*op(A)op(B)+beta*C on the uplo part (long double), C
    elsewhere (including the ld padding); absdot = sum_p |a*b|."""
    A, Ap = _f64(A if A is not None and len(A) else np.zeros(1))
    B, Bp = _f64(B if B is not None and len(B) else np.zeros(1))
    Cin, Cp = _f64(Cin)
    out = Cin.copy()
    absdot = np.zeros_like(Cin)
    lib().orc_gemm_ld(uplo, transA, transB, m, n, k, alpha, Ap, lda, Bp, ldb, beta, Cp, ldc,
                      out.ctypes.data_as(_f64p), ldc, absdot.ctypes.data_as(_f64p))
    return out, absdot


def sgemm_wgsl(uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, Cin, ldc):
    """The reference's fp32 per-element order; returns the updated C."""
    A, Ap = _f32(A if A is not None and len(A) else np.zeros(1))
    B, Bp = _f32(B if B is not None and len(B) else np.zeros(1))
    out = np.array(Cin, dtype=np.float32, copy=True)
    lib().orc_sgemm_wgsl(uplo, transA, transB, m, n, k, alpha, Ap, lda, Bp, ldb, beta,
                         out.ctypes.data_as(_f32p), ldc)
    return out


def ssyr2k_ld(uplo, trans, n, k, alpha, A, lda, B, ldb, beta, Cin, ldc):
    """Returns (out, absdot1, absdot2), (ldc*n)-long column-major: out holds
    alpha*(op(A)op(B)^T + op(B)op(A)^T) + beta*C on the uplo triangle (long
    double), C elsewhere; absdot1 / absdot2 the two products' sum_p |a*b|."""
    A, Ap = _f64(A if A is not None and len(A) else np.zeros(1))
    B, Bp = _f64(B if B is not None and len(B) else np.zeros(1))
    Cin, Cp = _f64(Cin)
    out = Cin.copy()
    a1, a2 = np.zeros_like(Cin), np.zeros_like(Cin)
    lib().orc_ssyr2k_ld(uplo, trans, n, k, alpha, Ap, lda, Bp, ldb, beta, Cp, ldc,
                        out.ctypes.data_as(_f64p), a1.ctypes.data_as(_f64p),
                        a2.ctypes.data_as(_f64p))
    return out, a1, a2


def ssymm_ld(side, uplo, m, n, alpha, A, lda, B, ldb, beta, Cin, ldc):
    """Returns (out, absdot): alpha*S*B + beta*C (side 1) or alpha*B*S +
    beta*C (side 2), S the symmetric matrix of A's uplo triangle."""
    A, Ap = _f64(A)
    B, Bp = _f64(B)
    Cin, Cp = _f64(Cin)
    out = Cin.copy()
    ad = np.zeros_like(Cin)
    lib().orc_ssymm_ld(side, uplo, m, n, alpha, Ap, lda, Bp, ldb, beta, Cp, ldc,
                       out.ctypes.data_as(_f64p), ad.ctypes.data_as(_f64p))
    return out, ad


def strmm_ld(side, uplo, trans, unit, m, n, alpha, A, lda, B, ldb):
    """Returns (out, absdot): alpha*op(A)*B (side 1) or alpha*B*op(A) (side
    2) over A's triangle, in B's layout (padding copied from B)."""
    A, Ap = _f64(A)
    B, Bp = _f64(B)
    out = B.copy()
    ad = np.zeros_like(B)
    lib().orc_strmm_ld(side, uplo, trans, unit, m, n, alpha, Ap, lda, Bp, ldb,
                       out.ctypes.data_as(_f64p), ad.ctypes.data_as(_f64p))
    return out, ad


def strsm_ld(side, uplo, trans, unit, m, n, alpha, A, lda, B, ldb):
    """X with op(A) X = alpha B (side 1) or X op(A) = alpha B (side 2), in B's
    layout (padding copied from B), by long-double substitution."""
    A, Ap = _f64(A)
    out = np.array(B, dtype=np.float64, copy=True)
    lib().orc_strsm_ld(side, uplo, trans, unit, m, n, alpha, Ap, lda,
                       out.ctypes.data_as(_f64p), ldb)
    return out


def sger_ld(m, n, alpha, x, incx, y, incy, A, lda):
    """Returns the whole updated A buffer: alpha x y^T + A in long double
    (reference BLAS's column order and zero-y skip), column-major."""
    x, xp = _f64(x if x is not None and len(x) else np.zeros(1))
    y, yp = _f64(y if y is not None and len(y) else np.zeros(1))
    out = np.array(A if A is not None and len(A) else np.zeros(1), dtype=np.float64, copy=True)
    lib().orc_sger_ld(m, n, alpha, xp, incx, yp, incy, out.ctypes.data_as(_f64p), lda)
    return out[: len(A)] if A is not None else out


def ssymv_ld(uplo, n, alpha, A, lda, x, incx, beta, y, incy):
    """Returns (y_out, absdot): y_out the whole updated y buffer (alpha S x +
    beta y in long double, S from A's uplo triangle; reference BLAS's
    rules), absdot per output element."""
    A, Ap = _f64(A if A is not None and len(A) else np.zeros(1))
    x, xp = _f64(x if x is not None and len(x) else np.zeros(1))
    out = np.array(y, dtype=np.float64, copy=True)
    ad = np.zeros(max(n, 1))
    lib().orc_ssymv_ld(uplo, n, alpha, Ap, lda, xp, incx, beta, out.ctypes.data_as(_f64p), incy,
                       ad.ctypes.data_as(_f64p))
    return out, ad


def strmv_ld(uplo, trans, unit, n, A, lda, x, incx, y, incy):
    """Returns (y_out, absdot): y_out the whole y buffer with op(T) x written
    to its strided slots (long double; T the uplo triangle of the
    column-major A, unit diagonal taken as 1, trans 0's column form skipping
    zero x entries), absdot per output element."""
    A, Ap = _f64(A if A is not None and len(A) else np.zeros(1))
    x, xp = _f64(x if x is not None and len(x) else np.zeros(1))
    out = np.array(y if len(y) else np.zeros(1), dtype=np.float64, copy=True)
    ad = np.zeros(max(n, 1))
    lib().orc_strmv_ld(uplo, trans, unit, n, Ap, lda, xp, incx, out.ctypes.data_as(_f64p), incy,
                       ad.ctypes.data_as(_f64p))
    return out, ad


def ssyr_ld(uplo, n, alpha, x, incx, A, lda):
    """The whole updated A buffer: the uplo triangle (1 lower, 2 upper) of
    alpha x x^T + A in long double (zero-x column skip), column-major."""
    return ssyr2_ld(uplo, n, alpha, x, incx, None, 1, A, lda)


def ssyr2_ld(uplo, n, alpha, x, incx, y, incy, A, lda):
    """ssyr2 (y given) or ssyr (y None): the uplo triangle of
    alpha x y^T + alpha y x^T + A in long double, column-major."""
    two = y is not None
    x, xp = _f64(x if x is not None and len(x) else np.zeros(1))
    y, yp = _f64(y if two and len(y) else np.zeros(1))
    out = np.array(A if len(A) else np.zeros(1), dtype=np.float64, copy=True)
    lib().orc_ssyr2_ld(uplo, n, alpha, xp, incx, yp, incy, int(two), out.ctypes.data_as(_f64p), lda)
    return out[: len(A)]


def sgemv_ld(trans, m, n, alpha, A, lda, x, incx, beta, y, incy):
    """Returns (y_out, absdot): y_out the whole updated y buffer (long double
    accumulation, reference BLAS's rules), absdot per output element."""
    A, Ap = _f64(A if A is not None and len(A) else np.zeros(1))
    x, xp = _f64(x if x is not None and len(x) else np.zeros(1))
    out = np.array(y, dtype=np.float64, copy=True)
    ln = max(n if trans else m, 1)
    ad = np.zeros(ln)
    lib().orc_sgemv_ld(trans, m, n, alpha, Ap, lda, xp, incx, beta, out.ctypes.data_as(_f64p), incy,
                       ad.ctypes.data_as(_f64p))
    return out, ad
