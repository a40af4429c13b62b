"""Builds libwgblas_hip.so (gfx950) and the Node-API addon, in-tree.

    python -m wgblas_amd.build            # both
    python -m wgblas_amd.build --lib      # the HIP library only

Outputs go to wgblas_amd/lib/. Every HIP translation unit is compiled with
packed-fp32 instructions disabled (-packed-fp32-ops): the compiler must not
emit v_pk_{add,mul,fma}_f32.
"""
import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
INCLUDE = os.path.join(ROOT, "include")

HIP_SOURCES = ["runtime.hip", "reduce.hip", "gemm.hip", "level3.hip", "level2.hip", "noalloc.hip"]
LIB_NAME = "libwgblas_hip.so"
ADDON_NAME = "wgblas_hip.node"
ARCH = os.environ.get("WGBLAS_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: a ROCm toolchain is required to build libwgblas_hip")
    return path


def _run(cmd):
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build_lib(verbose=False):
    os.makedirs(LIBDIR, exist_ok=True)
    objdir = os.path.join(LIBDIR, "obj")
    os.makedirs(objdir, exist_ok=True)
    hipcc = _hipcc()

    def compile_one(src):
        obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, "-I", INCLUDE, "-c", os.path.join(CSRC, src), "-o", obj]
        out = _run(cmd)
        if verbose and out.strip():
            print(out)
        return obj

    with cf.ThreadPoolExecutor(max_workers=len(HIP_SOURCES)) as ex:
        objs = list(ex.map(compile_one, HIP_SOURCES))
    out_path = os.path.join(LIBDIR, LIB_NAME)
    tmp = out_path + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, out_path)
    return out_path


def build_addon(verbose=False):
    """Node-API addon: plain host C++ against node_api.h, linked to the HIP library."""
    node_inc = None
    for cand in ("/usr/include/node", "/usr/local/include/node"):
        if os.path.exists(os.path.join(cand, "node_api.h")):
            node_inc = cand
            break
    if node_inc is None:
        raise RuntimeError("node_api.h not found: cannot build the Node-API addon")
    src = os.path.join(CSRC, "napi_addon.cc")
    out_path = os.path.join(LIBDIR, ADDON_NAME)
    tmp = out_path + ".tmp"
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
        "-I", node_inc, "-I", INCLUDE,
        "-DNAPI_VERSION=8",
        src, "-o", tmp,
        "-L", LIBDIR, "-lwgblas_hip", "-Wl,-rpath,$ORIGIN",
    ]
    out = _run(cmd)
    if verbose and out.strip():
        print(out)
    os.replace(tmp, out_path)
    return out_path


def build_twin(verbose=False):
    """The rocBLAS twin of bench.py's workloads (vendor context numbers):
    host code only, linked to rocBLAS and to libwgblas_hip for its seeded
    fills."""
    src = os.path.join(CSRC, "vendor_twin.cpp")
    out_path = os.path.join(LIBDIR, "vendor_twin")
    tmp = out_path + ".tmp"
    cmd = [
        _hipcc(), f"--offload-arch={ARCH}", "-O2", "-std=c++17",
        "-I", INCLUDE, src, "-o", tmp,
        "-L", LIBDIR, "-lwgblas_hip", "-lrocblas", "-Wl,-rpath,$ORIGIN",
    ]
    out = _run(cmd)
    if verbose and out.strip():
        print(out)
    os.replace(tmp, out_path)
    return out_path


def build_probe(verbose=False):
    """The roof probe (HBM read / copy bandwidth, fp32 / fp64 MFMA issue
    rate measured on the box; bench.py reports it beside the published
    peaks)."""
    src = os.path.join(CSRC, "roof_probe.hip")
    out_path = os.path.join(LIBDIR, "roof_probe")
    tmp = out_path + ".tmp"
    out = _run([_hipcc(), *HIPCC_FLAGS, src, "-o", tmp])
    if verbose and out.strip():
        print(out)
    os.replace(tmp, out_path)
    return out_path


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--lib", action="store_true", help="build only the HIP library")
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args(argv)
    lib = build_lib(args.verbose)
    print(f"built {lib}")
    if not args.lib:
        addon = build_addon(args.verbose)
        print(f"built {addon}")
        twin = build_twin(args.verbose)
        print(f"built {twin}")
        probe = build_probe(args.verbose)
        print(f"built {probe}")


if __name__ == "__main__":
    sys.exit(main())
