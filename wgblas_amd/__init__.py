"""wgblas_amd: MI355X (gfx950) HIP implementation of wgblas's GEMM family (and
the level-3 routines built on it) and level-1 reductions, behind a C ABI
(include/wgblas_hip.h).

  * wgblas_amd/csrc/   HIP kernels + the C ABI (libwgblas_hip.so)
  * wgblas_amd/js/     the wgblas JavaScript API over a Node-API addon
  * wgblas_amd.native  ctypes binding of the C ABI (tests, bench)
"""
from .native import (  # noqa: F401
    LEFT,
    LIB_PATH,
    LOWER,
    NO_TRANS,
    NON_UNIT,
    RIGHT,
    TRANS,
    UNIT,
    UPPER,
    Context,
    DeviceArray,
    WgblasError,
    device_count,
    exported_symbols,
    library,
)
