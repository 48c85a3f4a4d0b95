"""Builds liblrm_hip.so in-tree (rosylnalive_amd/liblrm_hip.so) for gfx950.

HIP sources are compiled by hipcc for gfx950 only, with packed-fp32 instructions disabled and no fp contraction
(every fused multiply-add in the kernels is written as fmaf); host sources by g++; the library is linked by g++
against libamdhip64. Objects go to rosylnalive_amd/_build/. Run: python -m rosylnalive_amd.build
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "liblrm_hip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIP_SOURCES = ["kernels_catalog.hip", "kernels_fast.hip", "kernels_persist.hip", "scratch_static.hip"]
HOST_SOURCES = ["contract.cpp", "device.cpp", "qwen_exec.cpp", "safetensors.cpp", "tokenizer.cpp", "capi.cpp"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
]
CXX_FLAGS = [
    "-O2",
    "-std=c++17",
    "-fPIC",
    "-fopenmp",
    "-D__HIP_PLATFORM_AMD__",
    "-I" + os.path.join(ROCM, "include"),
    "-Wall",
    "-Wextra",
    "-Wno-unused-parameter",
]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("build step failed:\n" + " ".join(cmd) + "\n" + r.stdout + r.stderr)
    return r.stderr


# The stage-timing variant of the library (the persistent decode step records constant-clock stamps at its stage
# boundaries; rosylnalive_amd/persist_stages.py reads them): same sources, built apart with LRM_PERSIST_STAMPS.
STAMPS_DIR = os.path.join(HERE, "stamps")
STAMPS_LIB = os.path.join(STAMPS_DIR, "liblrm_hip.so")


def build(verbose: bool = False, stamps: bool = False) -> str:
    hipcc = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    cxx = shutil.which("g++") or "g++"
    build_dir = os.path.join(STAMPS_DIR, "_build") if stamps else BUILD
    lib_path = STAMPS_LIB if stamps else LIB
    extra = ["-DLRM_PERSIST_STAMPS", "-DLRM_GEMM_STAMPS"] if stamps else []
    os.makedirs(build_dir, exist_ok=True)
    jobs = []
    for s in HIP_SOURCES:
        jobs.append([hipcc, *HIPCC_FLAGS, *extra, "-c", os.path.join(CSRC, s), "-o", os.path.join(build_dir, s + ".o")])
    for s in HOST_SOURCES:
        jobs.append([cxx, *CXX_FLAGS, *extra, "-c", os.path.join(CSRC, s), "-o", os.path.join(build_dir, s + ".o")])
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        for err in ex.map(_run, jobs):
            if verbose and err.strip():
                print(err, file=sys.stderr)
    objs = [os.path.join(build_dir, s + ".o") for s in HIP_SOURCES + HOST_SOURCES]
    tmp = lib_path + ".tmp"
    _run([cxx, "-shared", "-o", tmp, *objs, "-L" + os.path.join(ROCM, "lib"), "-Wl,-rpath," + os.path.join(ROCM, "lib"),
          "-lamdhip64", "-fopenmp", "-lquadmath"])
    os.replace(tmp, lib_path)
    return lib_path


if __name__ == "__main__":
    print(build(verbose=True, stamps="--stamps" in sys.argv[1:]))
