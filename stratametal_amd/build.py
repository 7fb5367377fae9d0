"""Build libsmoe.so (the HIP kernels + C ABI) for gfx950 with hipcc, in-tree.

    python -m stratametal_amd.build          # or __graft_entry__.build()

Objects go to stratametal_amd/_build/, the library to stratametal_amd/lib/libsmoe.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libsmoe.so")
DEMO = os.path.join(LIBDIR, "smoe_ffn_demo")  # the C++ operator (include/smoe_ffn.hpp) end to end, over libsmoe.so

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -ffp-contract=off: every fused multiply-add in the kernels is written as __builtin_fmaf, so the reduction
# orders the oracle restates are the ones that run.  Packed FP32 is disabled for correctness on this fleet.
COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    # MFMA results in VGPRs: the prefill kernels scale every block's MFMA result on the VALU, and in AGPRs
    # each element would first be copied out with v_accvgpr_read
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    # the first 14 dwords of every kernel's arguments arrive in SGPRs with the wave (gfx950 kernarg preloading;
    # the code object keeps a prologue that loads them itself where the firmware does not preload), so the
    # decode kernels issue their first loads without a scalar round trip to the argument buffer
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
    "-Wall", "-Wno-unused-result",
]

SOURCES = ["smoe_decode.hip", "smoe_prefill.hip", "smoe_iq2.hip", "smoe_hc.hip", "smoe_native.hip", "smoe_cache.hip",
           "smoe_synth.hip", "smoe_api.cpp", "smoe_gguf.cpp"]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *COMMON, "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    out = subprocess.run(cmd, capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{out.stderr}")
    return obj


# The host-sanitized library (AddressSanitizer + UndefinedBehaviorSanitizer on the host code of the C ABI and the
# GGUF reader; the kernels as built above): lib/libsmoe_asan.so, for tests/test_sanitize.py, which runs the CPU tests
# on it (and on a sanitized build of the test checker) under the clang sanitizer runtime.  Never loaded by the
# product path.
LIB_ASAN = os.path.join(LIBDIR, "libsmoe_asan.so")
HOST_SOURCES = ["smoe_api.cpp", "smoe_gguf.cpp"]
SANITIZE = [f for opt in ("-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=undefined",
                          "-fno-omit-frame-pointer") for f in ("-Xarch_host", opt)]


def _compile_asan(src: str) -> str:
    obj = os.path.join(BUILD, "asan", os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, "-x", "hip", *COMMON, *SANITIZE, "-c", os.path.join(CSRC, src), "-o", obj]
    out = subprocess.run(cmd, capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError(f"hipcc (sanitized host) failed on {src}:\n{out.stderr}")
    return obj


def build_sanitized(verbose: bool = False) -> str:
    """lib/libsmoe_asan.so from the kernel objects of build() and sanitized host objects."""
    os.makedirs(os.path.join(BUILD, "asan"), exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(HOST_SOURCES)) as ex:
        host = list(ex.map(_compile_asan, HOST_SOURCES))
    kern = [os.path.join(BUILD, os.path.splitext(s)[0] + ".o") for s in SOURCES if s not in HOST_SOURCES]
    tmp = LIB_ASAN + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-shared-libsan", *SANITIZE, "-o", tmp, *host, *kern]
    out = subprocess.run(cmd, capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError(f"sanitized link failed:\n{out.stderr}")
    os.replace(tmp, LIB_ASAN)
    if verbose:
        print("built", LIB_ASAN)
    return LIB_ASAN


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    out = subprocess.run(cmd, capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError(f"link failed:\n{out.stderr}")
    os.replace(tmp, LIB)
    cmd = [HIPCC, *COMMON, "-x", "hip", os.path.join(CSRC, "smoe_ffn_demo.cpp"), "-L", LIBDIR, "-lsmoe",
           "-Wl,-rpath,$ORIGIN", "-o", DEMO + ".tmp"]
    out = subprocess.run(cmd, capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError(f"smoe_ffn_demo failed:\n{out.stderr}")
    os.replace(DEMO + ".tmp", DEMO)
    if verbose:
        print("built", LIB, "and", DEMO)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
