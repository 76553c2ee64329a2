"""Build recipe for the native parts of nibblegemm_amd (in-tree, gfx950 only).

Produces:

* ``nibblegemm_amd/lib/libnibblegemm_amd.so`` -- the C-ABI library
  (``include/nibblegemm_amd.h``): HIP kernels + host validation, built with
  ``hipcc --offload-arch=gfx950``;
* ``nibblegemm_amd/_binding<EXT_SUFFIX>`` -- the CPython binding over that C ABI
  (plain C, built with gcc, no torch headers), loading the library through an
  ``$ORIGIN/lib`` rpath.

Run as ``python -m nibblegemm_amd.build`` or through ``__graft_entry__.build()``.
Every call recompiles.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJ = os.path.join(PKG, "_build")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libnibblegemm_amd.so")

HIP_SOURCES = ["abi.hip", "dequant.hip", "gemv.hip", "gemm.hip", "glue.hip", "chain.hip", "probe.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    # No packed-fp32 VALU ops (v_pk_add/mul/fma_f32) anywhere in device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Leading scalar kernel arguments (up to 14 dwords) arrive preloaded in
    # SGPRs instead of being fetched by each wave.
    "-mllvm", "-amdgpu-kernarg-preload-count=14",
    "-I", INCLUDE,
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = os.path.join(rocm, "bin", "hipcc")
    return cand if os.path.exists(cand) else (shutil.which("hipcc") or "hipcc")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def build_library(verbose: bool = False, jobs: int = 8) -> str:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    hipcc = _hipcc()

    def compile_one(src):
        obj = os.path.join(OBJ, src.replace(".hip", ".o"))
        _run([hipcc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj], verbose)
        return obj

    with cf.ThreadPoolExecutor(max_workers=min(jobs, len(HIP_SOURCES))) as ex:
        objs = list(ex.map(compile_one, HIP_SOURCES))
    tmp = LIB + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB)
    return LIB


def build_binding(verbose: bool = False) -> str:
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = os.path.join(PKG, "_binding" + suffix)
    py_inc = sysconfig.get_paths()["include"]
    tmp = out + ".tmp"
    _run([
        os.environ.get("CC", "gcc"), "-O2", "-fPIC", "-shared", "-std=c11", "-Wall",
        "-I", py_inc, "-I", INCLUDE,
        os.path.join(CSRC, "binding.c"),
        "-L", LIBDIR, "-lnibblegemm_amd",
        "-Wl,-rpath,$ORIGIN/lib",
        "-o", tmp,
    ], verbose)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> None:
    build_library(verbose)
    build_binding(verbose)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built", LIB)
