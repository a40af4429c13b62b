"""ctypes binding of libwgblas_hip's C ABI (include/wgblas_hip.h).

This is the Python view of the same boundary the Node-API addon binds: plain
pointers and sizes, column-major matrices, status codes turned into
WgblasError. It loads the in-tree library built by `python -m wgblas_amd.build`
and raises if it is missing: there is no CPU fallback.
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# WGBLAS_HIP_LIB points the binding at another build of the library.
LIB_PATH = os.environ.get("WGBLAS_HIP_LIB") or os.path.join(_HERE, "lib", "libwgblas_hip.so")

NO_TRANS, TRANS = 0, 1
LOWER, UPPER = 1, 2
LEFT, RIGHT = 1, 2
NON_UNIT, UNIT = 0, 1

_i64 = C.c_int64
_ptr = C.c_void_p

# name -> argtypes (every entry point returns int status unless listed in _RESTYPES)
_SIGNATURES = {
    "wgb_init": [C.c_int, C.POINTER(_ptr)],
    "wgb_destroy": [_ptr],
    "wgb_device_name": [_ptr, C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t],
    "wgb_device_count": [C.POINTER(C.c_int)],
    "wgb_set_timing": [_ptr, C.c_int],
    "wgb_last_time_ms": [_ptr, C.POINTER(C.c_float)],
    "wgb_synchronize": [_ptr],
    "wgb_stream": [_ptr],
    "wgb_last_error": [],
    "wgb_abi_version": [],
    "wgb_status_string": [C.c_int],
    "wgb_malloc": [_ptr, C.c_size_t, C.POINTER(_ptr)],
    "wgb_free": [_ptr, _ptr],
    "wgb_memcpy_h2d": [_ptr, _ptr, _ptr, C.c_size_t],
    "wgb_memcpy_d2h": [_ptr, _ptr, _ptr, C.c_size_t],
    "wgb_memcpy_d2d": [_ptr, _ptr, _ptr, C.c_size_t],
    "wgb_fill_uniform_f32": [_ptr, _ptr, _i64, C.c_double, C.c_double, C.c_uint32],
    "wgb_fill_uniform_f64": [_ptr, _ptr, _i64, C.c_double, C.c_double, C.c_uint32],
    "wgb_fill_normal_f32": [_ptr, _ptr, _i64, C.c_uint32],
    "wgb_sgemm": [_ptr, C.c_int, C.c_int, _i64, _i64, _i64, C.c_float, _ptr, _i64, _ptr, _i64,
                  C.c_float, _ptr, _i64],
    "wgb_sgemm_noalloc": [_ptr, C.c_int, C.c_int, _i64, _i64, _i64, C.c_float, _ptr, _i64, _ptr,
                          _i64, C.c_float, _ptr, _i64],
    "wgb_sgemmtr": [_ptr, C.c_int, C.c_int, C.c_int, _i64, _i64, _i64, C.c_float, _ptr, _i64,
                    _ptr, _i64, C.c_float, _ptr, _i64],
    "wgb_ssyrk": [_ptr, C.c_int, C.c_int, _i64, _i64, C.c_float, _ptr, _i64, C.c_float, _ptr,
                  _i64],
    "wgb_dgemm": [_ptr, C.c_int, C.c_int, _i64, _i64, _i64, C.c_double, _ptr, _i64, _ptr, _i64,
                  C.c_double, _ptr, _i64],
    "wgb_dgemmtr": [_ptr, C.c_int, C.c_int, C.c_int, _i64, _i64, _i64, C.c_double, _ptr, _i64,
                    _ptr, _i64, C.c_double, _ptr, _i64],
    "wgb_dsyrk": [_ptr, C.c_int, C.c_int, _i64, _i64, C.c_double, _ptr, _i64, C.c_double, _ptr,
                  _i64],
    "wgb_ssyr2k": [_ptr, C.c_int, C.c_int, C.c_int, _i64, _i64, C.c_float, _ptr, _i64, _ptr, _i64,
                   C.c_float, _ptr, _i64],
    "wgb_ssymm": [_ptr, C.c_int, C.c_int, C.c_int, _i64, _i64, C.c_float, _ptr, _i64, _ptr, _i64,
                  C.c_float, _ptr, _i64],
    "wgb_strmm": [_ptr, C.c_int, C.c_int, C.c_int, C.c_int, _i64, _i64, C.c_float, _ptr, _i64,
                  _ptr, _i64],
    "wgb_dsyr2k": [_ptr, C.c_int, C.c_int, C.c_int, _i64, _i64, C.c_double, _ptr, _i64, _ptr, _i64,
                   C.c_double, _ptr, _i64],
    "wgb_dsymm": [_ptr, C.c_int, C.c_int, C.c_int, _i64, _i64, C.c_double, _ptr, _i64, _ptr, _i64,
                  C.c_double, _ptr, _i64],
    "wgb_dtrmm": [_ptr, C.c_int, C.c_int, C.c_int, C.c_int, _i64, _i64, C.c_double, _ptr, _i64,
                  _ptr, _i64],
    "wgb_strsm": [_ptr, C.c_int, C.c_int, C.c_int, C.c_int, _i64, _i64, C.c_float, _ptr, _i64,
                  _ptr, _i64],
    "wgb_sgemv": [_ptr, C.c_int, _i64, _i64, C.c_float, _ptr, _i64, _ptr, _i64, C.c_float, _ptr,
                  _i64],
    "wgb_sger": [_ptr, _i64, _i64, C.c_float, _ptr, _i64, _ptr, _i64, _ptr, _i64],
    "wgb_dger": [_ptr, _i64, _i64, C.c_double, _ptr, _i64, _ptr, _i64, _ptr, _i64],
    "wgb_ssyr": [_ptr, C.c_int, _i64, C.c_float, _ptr, _i64, _ptr, _i64],
    "wgb_dsyr": [_ptr, C.c_int, _i64, C.c_double, _ptr, _i64, _ptr, _i64],
    "wgb_ssyr2": [_ptr, C.c_int, _i64, C.c_float, _ptr, _i64, _ptr, _i64, _ptr, _i64],
    "wgb_dsyr2": [_ptr, C.c_int, _i64, C.c_double, _ptr, _i64, _ptr, _i64, _ptr, _i64],
    "wgb_strmv": [_ptr, C.c_int, C.c_int, C.c_int, _i64, _ptr, _i64, _ptr, _i64, _ptr, _i64],
    "wgb_dtrmv": [_ptr, C.c_int, C.c_int, C.c_int, _i64, _ptr, _i64, _ptr, _i64, _ptr, _i64],
    "wgb_ssymv": [_ptr, C.c_int, _i64, C.c_float, _ptr, _i64, _ptr, _i64, C.c_float, _ptr, _i64],
    "wgb_dsymv": [_ptr, C.c_int, _i64, C.c_double, _ptr, _i64, _ptr, _i64, C.c_double, _ptr, _i64],
    "wgb_dgemv": [_ptr, C.c_int, _i64, _i64, C.c_double, _ptr, _i64, _ptr, _i64, C.c_double, _ptr,
                  _i64],
    "wgb_sdot": [_ptr, _i64, _ptr, _i64, _ptr, _i64, C.POINTER(C.c_float)],
    "wgb_sdot_dev": [_ptr, _i64, _ptr, _i64, _ptr, _i64, _ptr],
    "wgb_sasum": [_ptr, _i64, _ptr, _i64, C.POINTER(C.c_float)],
    "wgb_sasum_dev": [_ptr, _i64, _ptr, _i64, _ptr],
    "wgb_snrm2": [_ptr, _i64, _ptr, _i64, C.POINTER(C.c_float)],
    "wgb_snrm2_dev": [_ptr, _i64, _ptr, _i64, _ptr],
    "wgb_isamax": [_ptr, _i64, _ptr, _i64, C.POINTER(_i64)],
    "wgb_isamax_dev": [_ptr, _i64, _ptr, _i64, _ptr],
    "wgb_ddot": [_ptr, _i64, _ptr, _i64, _ptr, _i64, C.POINTER(C.c_double)],
    "wgb_ddot_dev": [_ptr, _i64, _ptr, _i64, _ptr, _i64, _ptr],
    "wgb_dasum": [_ptr, _i64, _ptr, _i64, C.POINTER(C.c_double)],
    "wgb_dasum_dev": [_ptr, _i64, _ptr, _i64, _ptr],
    "wgb_dnrm2": [_ptr, _i64, _ptr, _i64, C.POINTER(C.c_double)],
    "wgb_dnrm2_dev": [_ptr, _i64, _ptr, _i64, _ptr],
    "wgb_idamax": [_ptr, _i64, _ptr, _i64, C.POINTER(_i64)],
    "wgb_idamax_dev": [_ptr, _i64, _ptr, _i64, _ptr],
}
_RESTYPES = {
    "wgb_stream": _ptr,
    "wgb_last_error": C.c_char_p,
    "wgb_status_string": C.c_char_p,
}

_lib = None

# WGB_ABI_VERSION of include/wgblas_hip.h that these signatures follow.
ABI_VERSION = 3


class WgblasError(RuntimeError):
    def __init__(self, status, where, message):
        super().__init__(f"{where} failed with status {status}: {message}")
        self.status = status


def library():
    """Loads libwgblas_hip.so once; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m wgblas_amd.build` "
                "(the HIP library is required; there is no CPU fallback)")
        lib = C.CDLL(LIB_PATH)
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, C.c_int)
        if lib.wgb_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} implements C ABI version {lib.wgb_abi_version()}, this binding "
                               f"expects {ABI_VERSION}: rebuild with `python -m wgblas_amd.build`")
        _lib = lib
    return _lib


def exported_symbols():
    return sorted(_SIGNATURES)


def _check(status, where):
    if status != 0:
        msg = library().wgb_last_error().decode(errors="replace")
        raise WgblasError(status, where, msg)


def device_count():
    c = C.c_int(0)
    _check(library().wgb_device_count(C.byref(c)), "wgb_device_count")
    return c.value


class DeviceArray:
    """A device allocation with a numpy dtype and shape (no layout implied)."""

    def __init__(self, ctx, ptr, nbytes, dtype, shape):
        self.ctx, self.ptr, self.nbytes = ctx, ptr, nbytes
        self.dtype, self.shape = np.dtype(dtype), tuple(shape)

    @property
    def size(self):
        return int(np.prod(self.shape, dtype=np.int64))

    def offset(self, elems):
        """Raw pointer `elems` elements into the allocation (no bounds kept)."""
        return self.ptr + int(elems) * self.dtype.itemsize

    def to_host(self):
        out = np.empty(self.shape, dtype=self.dtype)
        if out.nbytes:
            self.ctx.d2h(out, self.ptr)
        return out

    def free(self):
        if self.ptr:
            self.ctx.free(self.ptr)
            self.ptr = 0


class Context:
    """One HIP device and stream (wgb_ctx)."""

    def __init__(self, device=0):
        self.lib = library()
        h = _ptr()
        _check(self.lib.wgb_init(device, C.byref(h)), "wgb_init")
        self.handle = h.value
        self.device = device

    def close(self):
        if self.handle:
            self.lib.wgb_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- device info / timing ----
    def name(self):
        name = C.create_string_buffer(256)
        arch = C.create_string_buffer(64)
        _check(self.lib.wgb_device_name(self.handle, name, 256, arch, 64), "wgb_device_name")
        return name.value.decode(), arch.value.decode()

    @property
    def stream(self):
        return self.lib.wgb_stream(self.handle)

    def set_timing(self, on):
        _check(self.lib.wgb_set_timing(self.handle, 1 if on else 0), "wgb_set_timing")

    def last_time_ms(self):
        ms = C.c_float(0)
        _check(self.lib.wgb_last_time_ms(self.handle, C.byref(ms)), "wgb_last_time_ms")
        return ms.value

    def synchronize(self):
        _check(self.lib.wgb_synchronize(self.handle), "wgb_synchronize")

    # ---- memory ----
    def malloc(self, nbytes):
        p = _ptr()
        _check(self.lib.wgb_malloc(self.handle, int(nbytes), C.byref(p)), "wgb_malloc")
        return p.value

    def free(self, ptr):
        _check(self.lib.wgb_free(self.handle, ptr), "wgb_free")

    def h2d(self, dst_ptr, host):
        host = np.ascontiguousarray(host)
        _check(self.lib.wgb_memcpy_h2d(self.handle, dst_ptr, host.ctypes.data, host.nbytes),
               "wgb_memcpy_h2d")

    def d2h(self, host, src_ptr):
        assert host.flags.c_contiguous
        _check(self.lib.wgb_memcpy_d2h(self.handle, host.ctypes.data, src_ptr, host.nbytes),
               "wgb_memcpy_d2h")

    def empty(self, shape, dtype):
        shape = (shape,) if np.isscalar(shape) else tuple(shape)
        dt = np.dtype(dtype)
        nbytes = int(np.prod(shape, dtype=np.int64)) * dt.itemsize
        return DeviceArray(self, self.malloc(nbytes), nbytes, dt, shape)

    def upload(self, host):
        host = np.ascontiguousarray(host)
        arr = self.empty(host.shape, host.dtype)
        if host.nbytes:
            self.h2d(arr.ptr, host)
        return arr

    # ---- seeded inputs ----
    def fill_uniform(self, arr, low, high, seed, n=None):
        n = arr.size if n is None else n
        fn = {np.float32: self.lib.wgb_fill_uniform_f32,
              np.float64: self.lib.wgb_fill_uniform_f64}[arr.dtype.type]
        _check(fn(self.handle, arr.ptr, n, float(low), float(high), seed & 0xffffffff),
               "wgb_fill_uniform")

    def fill_normal(self, arr, seed, n=None):
        assert arr.dtype == np.float32
        n = arr.size if n is None else n
        _check(self.lib.wgb_fill_normal_f32(self.handle, arr.ptr, n, seed & 0xffffffff),
               "wgb_fill_normal_f32")

    # ---- level 3 (column-major, device pointers) ----
    def sgemm(self, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C_, ldc):
        _check(self.lib.wgb_sgemm(self.handle, transA, transB, m, n, k, alpha, _p(A), lda,
                                  _p(B), ldb, beta, _p(C_), ldc), "wgb_sgemm")

    def sgemm_noalloc(self, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C_, ldc):
        _check(self.lib.wgb_sgemm_noalloc(self.handle, transA, transB, m, n, k, alpha, _p(A), lda,
                                          _p(B), ldb, beta, _p(C_), ldc), "wgb_sgemm_noalloc")

    def sgemmtr(self, uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C_, ldc):
        _check(self.lib.wgb_sgemmtr(self.handle, uplo, transA, transB, m, n, k, alpha, _p(A),
                                    lda, _p(B), ldb, beta, _p(C_), ldc), "wgb_sgemmtr")

    def ssyrk(self, uplo, trans, n, k, alpha, A, lda, beta, C_, ldc):
        _check(self.lib.wgb_ssyrk(self.handle, uplo, trans, n, k, alpha, _p(A), lda, beta,
                                  _p(C_), ldc), "wgb_ssyrk")

    def dgemm(self, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C_, ldc):
        _check(self.lib.wgb_dgemm(self.handle, transA, transB, m, n, k, alpha, _p(A), lda,
                                  _p(B), ldb, beta, _p(C_), ldc), "wgb_dgemm")

    def dgemmtr(self, uplo, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C_, ldc):
        _check(self.lib.wgb_dgemmtr(self.handle, uplo, transA, transB, m, n, k, alpha, _p(A),
                                    lda, _p(B), ldb, beta, _p(C_), ldc), "wgb_dgemmtr")

    def dsyrk(self, uplo, trans, n, k, alpha, A, lda, beta, C_, ldc):
        _check(self.lib.wgb_dsyrk(self.handle, uplo, trans, n, k, alpha, _p(A), lda, beta,
                                  _p(C_), ldc), "wgb_dsyrk")

    def ssyr2k(self, uplo, trans, n, k, alpha, A, lda, B, ldb, beta, C_, ldc, transB=None):
        """`trans` applies to A, and to B unless `transB` is given."""
        tb = trans if transB is None else transB
        _check(self.lib.wgb_ssyr2k(self.handle, uplo, trans, tb, n, k, alpha, _p(A), lda, _p(B),
                                   ldb, beta, _p(C_), ldc), "wgb_ssyr2k")

    def ssymm(self, side, uplo, m, n, alpha, A, lda, B, ldb, beta, C_, ldc, transB=NO_TRANS):
        _check(self.lib.wgb_ssymm(self.handle, side, uplo, transB, m, n, alpha, _p(A), lda, _p(B),
                                  ldb, beta, _p(C_), ldc), "wgb_ssymm")

    def strmm(self, side, uplo, transA, diag, m, n, alpha, A, lda, B, ldb):
        _check(self.lib.wgb_strmm(self.handle, side, uplo, transA, diag, m, n, alpha, _p(A), lda,
                                  _p(B), ldb), "wgb_strmm")

    def dsyr2k(self, uplo, trans, n, k, alpha, A, lda, B, ldb, beta, C_, ldc, transB=None):
        """`trans` applies to A, and to B unless `transB` is given."""
        tb = trans if transB is None else transB
        _check(self.lib.wgb_dsyr2k(self.handle, uplo, trans, tb, n, k, alpha, _p(A), lda, _p(B),
                                   ldb, beta, _p(C_), ldc), "wgb_dsyr2k")

    def dsymm(self, side, uplo, m, n, alpha, A, lda, B, ldb, beta, C_, ldc, transB=NO_TRANS):
        _check(self.lib.wgb_dsymm(self.handle, side, uplo, transB, m, n, alpha, _p(A), lda, _p(B),
                                  ldb, beta, _p(C_), ldc), "wgb_dsymm")

    def dtrmm(self, side, uplo, transA, diag, m, n, alpha, A, lda, B, ldb):
        _check(self.lib.wgb_dtrmm(self.handle, side, uplo, transA, diag, m, n, alpha, _p(A), lda,
                                  _p(B), ldb), "wgb_dtrmm")

    def strsm(self, side, uplo, transA, diag, m, n, alpha, A, lda, B, ldb):
        _check(self.lib.wgb_strsm(self.handle, side, uplo, transA, diag, m, n, alpha, _p(A), lda,
                                  _p(B), ldb), "wgb_strsm")

    # ---- level 2 ----
    def sgemv(self, trans, m, n, alpha, A, lda, x, incx, beta, y, incy):
        _check(self.lib.wgb_sgemv(self.handle, trans, m, n, alpha, _p(A), lda, _p(x), incx, beta,
                                  _p(y), incy), "wgb_sgemv")

    def sger(self, m, n, alpha, x, incx, y, incy, A, lda):
        _check(self.lib.wgb_sger(self.handle, m, n, alpha, _p(x), incx, _p(y), incy, _p(A), lda),
               "wgb_sger")

    def dger(self, m, n, alpha, x, incx, y, incy, A, lda):
        _check(self.lib.wgb_dger(self.handle, m, n, alpha, _p(x), incx, _p(y), incy, _p(A), lda),
               "wgb_dger")

    def ssyr(self, uplo, n, alpha, x, incx, A, lda):
        _check(self.lib.wgb_ssyr(self.handle, uplo, n, alpha, _p(x), incx, _p(A), lda), "wgb_ssyr")

    def dsyr(self, uplo, n, alpha, x, incx, A, lda):
        _check(self.lib.wgb_dsyr(self.handle, uplo, n, alpha, _p(x), incx, _p(A), lda), "wgb_dsyr")

    def ssyr2(self, uplo, n, alpha, x, incx, y, incy, A, lda):
        _check(self.lib.wgb_ssyr2(self.handle, uplo, n, alpha, _p(x), incx, _p(y), incy, _p(A), lda),
               "wgb_ssyr2")

    def dsyr2(self, uplo, n, alpha, x, incx, y, incy, A, lda):
        _check(self.lib.wgb_dsyr2(self.handle, uplo, n, alpha, _p(x), incx, _p(y), incy, _p(A), lda),
               "wgb_dsyr2")

    def ssymv(self, uplo, n, alpha, A, lda, x, incx, beta, y, incy):
        _check(self.lib.wgb_ssymv(self.handle, uplo, n, alpha, _p(A), lda, _p(x), incx, beta, _p(y), incy),
               "wgb_ssymv")

    def dsymv(self, uplo, n, alpha, A, lda, x, incx, beta, y, incy):
        _check(self.lib.wgb_dsymv(self.handle, uplo, n, alpha, _p(A), lda, _p(x), incx, beta, _p(y), incy),
               "wgb_dsymv")

    def strmv(self, uplo, trans, diag, n, A, lda, x, incx, y, incy):
        _check(self.lib.wgb_strmv(self.handle, uplo, trans, diag, n, _p(A), lda, _p(x), incx, _p(y), incy),
               "wgb_strmv")

    def dtrmv(self, uplo, trans, diag, n, A, lda, x, incx, y, incy):
        _check(self.lib.wgb_dtrmv(self.handle, uplo, trans, diag, n, _p(A), lda, _p(x), incx, _p(y), incy),
               "wgb_dtrmv")

    def dgemv(self, trans, m, n, alpha, A, lda, x, incx, beta, y, incy):
        _check(self.lib.wgb_dgemv(self.handle, trans, m, n, alpha, _p(A), lda, _p(x), incx, beta,
                                  _p(y), incy), "wgb_dgemv")

    # ---- level 1 ----
    def sdot(self, n, x, incx, y, incy):
        r = C.c_float(0)
        _check(self.lib.wgb_sdot(self.handle, n, _p(x), incx, _p(y), incy, C.byref(r)),
               "wgb_sdot")
        return np.float32(r.value)

    def sdot_dev(self, n, x, incx, y, incy, out):
        _check(self.lib.wgb_sdot_dev(self.handle, n, _p(x), incx, _p(y), incy, _p(out)),
               "wgb_sdot_dev")

    def sasum(self, n, x, incx):
        r = C.c_float(0)
        _check(self.lib.wgb_sasum(self.handle, n, _p(x), incx, C.byref(r)), "wgb_sasum")
        return np.float32(r.value)

    def sasum_dev(self, n, x, incx, out):
        _check(self.lib.wgb_sasum_dev(self.handle, n, _p(x), incx, _p(out)), "wgb_sasum_dev")

    def snrm2(self, n, x, incx):
        r = C.c_float(0)
        _check(self.lib.wgb_snrm2(self.handle, n, _p(x), incx, C.byref(r)), "wgb_snrm2")
        return np.float32(r.value)

    def snrm2_dev(self, n, x, incx, out):
        _check(self.lib.wgb_snrm2_dev(self.handle, n, _p(x), incx, _p(out)), "wgb_snrm2_dev")

    def isamax(self, n, x, incx):
        r = _i64(0)
        _check(self.lib.wgb_isamax(self.handle, n, _p(x), incx, C.byref(r)), "wgb_isamax")
        return int(r.value)

    def isamax_dev(self, n, x, incx, out):
        _check(self.lib.wgb_isamax_dev(self.handle, n, _p(x), incx, _p(out)), "wgb_isamax_dev")

    # ---- fp64 level 1 ----
    def ddot(self, n, x, incx, y, incy):
        r = C.c_double(0)
        _check(self.lib.wgb_ddot(self.handle, n, _p(x), incx, _p(y), incy, C.byref(r)),
               "wgb_ddot")
        return float(r.value)

    def ddot_dev(self, n, x, incx, y, incy, out):
        _check(self.lib.wgb_ddot_dev(self.handle, n, _p(x), incx, _p(y), incy, _p(out)),
               "wgb_ddot_dev")

    def dasum(self, n, x, incx):
        r = C.c_double(0)
        _check(self.lib.wgb_dasum(self.handle, n, _p(x), incx, C.byref(r)), "wgb_dasum")
        return float(r.value)

    def dasum_dev(self, n, x, incx, out):
        _check(self.lib.wgb_dasum_dev(self.handle, n, _p(x), incx, _p(out)), "wgb_dasum_dev")

    def dnrm2(self, n, x, incx):
        r = C.c_double(0)
        _check(self.lib.wgb_dnrm2(self.handle, n, _p(x), incx, C.byref(r)), "wgb_dnrm2")
        return float(r.value)

    def dnrm2_dev(self, n, x, incx, out):
        _check(self.lib.wgb_dnrm2_dev(self.handle, n, _p(x), incx, _p(out)), "wgb_dnrm2_dev")

    def idamax(self, n, x, incx):
        r = _i64(0)
        _check(self.lib.wgb_idamax(self.handle, n, _p(x), incx, C.byref(r)), "wgb_idamax")
        return int(r.value)

    def idamax_dev(self, n, x, incx, out):
        _check(self.lib.wgb_idamax_dev(self.handle, n, _p(x), incx, _p(out)), "wgb_idamax_dev")


def _p(x):
    """Device pointer of a DeviceArray, or a raw integer pointer / None."""
    if x is None:
        return None
    if isinstance(x, DeviceArray):
        return x.ptr
    return int(x)
