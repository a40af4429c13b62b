"""The C ABI library loads, exports every entry point include/wgblas_hip.h
declares, and rejects bad arguments before touching a device. No compute
call is made here (this suite runs without a GPU)."""
import ctypes as C
import os
import re
import subprocess

import pytest

from wgblas_amd import native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "wgblas_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wgb_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_path():
    names = declared_functions()
    for required in ["wgb_init", "wgb_destroy", "wgb_malloc", "wgb_free", "wgb_memcpy_h2d",
                     "wgb_memcpy_d2h", "wgb_sgemm", "wgb_sgemmtr", "wgb_ssyrk", "wgb_dgemm",
                     "wgb_sdot", "wgb_sasum", "wgb_snrm2", "wgb_isamax"]:
        assert required in names


def test_abi_version_matches_the_header_and_the_binding():
    text = open(HEADER).read()
    version = int(re.search(r"#define WGB_ABI_VERSION (\d+)", text).group(1))
    assert native.library().wgb_abi_version() == version == native.ABI_VERSION
    addon = open(os.path.join(ROOT, "wgblas_amd", "csrc", "napi_addon.cc")).read()
    assert "wgb_abi_version() != WGB_ABI_VERSION" in addon


def test_library_exports_every_declared_symbol():
    lib = native.library()
    out = subprocess.run(["nm", "-D", "--defined-only", native.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (wgb_[a-z0-9_]+)$", out, flags=re.M))
    for name in declared_functions():
        assert name in exported, name
        assert getattr(lib, name) is not None
    # the ctypes binding covers exactly the declared surface
    assert set(native.exported_symbols()) == set(declared_functions())


def test_library_has_gfx950_code_object():
    out = subprocess.run(["strings", native.LIB_PATH], capture_output=True, text=True).stdout
    assert "gfx950" in out


def test_status_strings_and_null_context():
    lib = native.library()
    assert lib.wgb_status_string(0) == b"ok"
    assert lib.wgb_status_string(-1) == b"invalid value"
    # a null context is rejected before any HIP call
    st = lib.wgb_sgemm(None, 0, 0, 2, 2, 2, 1.0, None, 2, None, 2, 0.0, None, 2)
    assert st == -5
    assert b"wgb_init" in lib.wgb_last_error()
    st = lib.wgb_sgemm_noalloc(None, 0, 0, 2, 2, 2, 1.0, None, 2, None, 2, 0.0, None, 2)
    assert st == -5
    r = C.c_float(1.0)
    assert lib.wgb_sdot(None, 4, None, 1, None, 1, C.byref(r)) == -5


def test_device_count_without_gpu_is_not_an_error():
    n = native.device_count()
    assert n >= 0


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(native, "LIB_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(native, "_lib", None)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        native.library()
