"""Build recipe for libung_hip.so (gfx950) -- run by __graft_entry__.build().

The library is built in-tree (filtervectorcode_refactor_amd/libung_hip.so) so it
travels with the repository snapshot to the GPU box:
  * ung_host.cpp    -> g++ (host C++: synthetic inputs, groups, LNG, reorder)
  * ung_runtime.hip -> hipcc --offload-arch=gfx950 (context, planning, launches, C ABI;
                       includes ung_kernels.hip, the device code: one translation unit)
Packed-FP32 instruction selection is disabled for all device code.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB_NAME = "libung_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
ARCH = os.environ.get("UNG_HIP_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")

HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-march=x86-64-v3", "-ffp-contract=off",
              "-Wall", "-Wextra", "-Wno-unused-parameter", "-pthread"]
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wno-unused-result", "-munsafe-fp-atomics"]


def _run(cmd, verbose):
    if verbose:
        print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}")
    elif verbose and (r.stderr.strip()):
        # keep warnings visible but short
        lines = [l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l]
        if lines:
            sys.stderr.write("\n".join(lines[:40]) + "\n")


def build(verbose: bool = True) -> str:
    """Compile libung_hip.so for gfx950; returns the library path."""
    obj_dir = os.path.join(HERE, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    host_obj = os.path.join(obj_dir, "ung_host.o")
    _run([CXX, *HOST_FLAGS, "-I", INCLUDE, "-I", CSRC, "-c",
          os.path.join(CSRC, "ung_host.cpp"), "-o", host_obj], verbose)
    dev_obj = os.path.join(obj_dir, "ung_runtime.o")
    _run([HIPCC, *HIP_FLAGS, "-I", INCLUDE, "-I", CSRC, "-c",
          os.path.join(CSRC, "ung_runtime.hip"), "-o", dev_obj], verbose)
    tmp = LIB_PATH + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", dev_obj, host_obj,
          "-o", tmp, "-pthread"], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


ADAPTER_SRC = os.path.join(ROOT, "tests", "cpp", "adapter_check.cpp")
ADAPTER_BIN = os.path.join(ROOT, "tests", "cpp", "_bin", "adapter_check")


def build_adapter_check(verbose: bool = True) -> str:
    """The C++ program that drives include/ung_hip_adapter.hpp against libung_hip.so
    (run by tests/test_gpu_adapter.py); linked with a relative run path so the tree can
    move to another machine."""
    os.makedirs(os.path.dirname(ADAPTER_BIN), exist_ok=True)
    tmp = ADAPTER_BIN + ".tmp"
    _run([CXX, "-std=c++17", "-O2", "-Wall", "-I", INCLUDE, ADAPTER_SRC, "-L", HERE, "-lung_hip",
          "-Wl,-rpath,$ORIGIN/../../../filtervectorcode_refactor_amd", "-Wl,-rpath-link,/opt/rocm/lib",
          "-o", tmp], verbose)
    os.replace(tmp, ADAPTER_BIN)
    return ADAPTER_BIN


if __name__ == "__main__":
    print(build(verbose=True))
