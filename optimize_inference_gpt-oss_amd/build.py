"""Builds libgkv.so (HIP kernels for gfx950 + host C++ + the C ABI) in-tree.

    python optimize_inference_gpt-oss_amd/build.py

hipcc compiles each source to an object (in parallel), then links one shared
library next to this file. Device code is built with packed-FP32 instruction
selection switched off (-Xclang -target-feature -Xclang -packed-fp32-ops);
the host pass warns that it does not know that feature, which is harmless.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libgkv.so")
DEMO = os.path.join(ROOT, "tests", "gkv_engine_demo")  # test driver of the C++ shim
EXPF_CHECK = os.path.join(ROOT, "tests", "gkv_expf_check")  # test driver of the exact expf

SOURCES = [
    "kv_append.hip",
    "decode_attention.hip",
    "prefill_attention.hip",
    "qkv_append.hip",
    "yardstick.hip",
    "exact_attention.hip",
    "rope_table.cpp",
    "kv_pool.cpp",
    "capi.cpp",
]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
COMMON = ["-std=c++17", "-O3", "-fPIC", "-Wall", "-I", os.path.join(ROOT, "include"), "-I", CSRC]
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    path = os.path.join(CSRC, src)
    # Every source, the host-only .cpp files included, compiles in HIP mode:
    # rope_table.cpp must round like the reference's own hipcc build of
    # run.cpp (HIP mode contracts a*b+c into FMAs, plain C++ mode does not),
    # and the others use the HIP runtime headers either way.
    cmd = [HIPCC, *COMMON, "-x", "hip", *DEVICE, "-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    # the C++ engine-shim test driver (tests/engine_demo.cpp): host code only,
    # linked against libgkv.so
    cmd = [HIPCC, "-std=c++17", "-O2", "-x", "c++", "-D__HIP_PLATFORM_AMD__", "-I", "/opt/rocm/include", "-I",
           os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "engine_demo.cpp"), "-o",
           DEMO + ".tmp", "-L", HERE, "-lgkv", "-Wl,-rpath,$ORIGIN/../optimize_inference_gpt-oss_amd"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"engine demo build failed:\n{r.stderr}")
    os.replace(DEMO + ".tmp", DEMO)
    # the exhaustive check of the exact path's expf against the host C library
    # (tests/expf_check.cpp): host code only, the header the kernels include
    cmd = [HIPCC, "-std=c++17", "-O2", "-x", "c++", "-D__HIP_PLATFORM_AMD__", "-I", "/opt/rocm/include",
           "-I", CSRC, "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "expf_check.cpp"),
           "-o", EXPF_CHECK + ".tmp", "-pthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"expf check build failed:\n{r.stderr}")
    os.replace(EXPF_CHECK + ".tmp", EXPF_CHECK)
    if verbose:
        print(f"built {LIB}, {DEMO} and {EXPF_CHECK}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
