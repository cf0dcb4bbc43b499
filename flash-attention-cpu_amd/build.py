"""Build the MI355X library in-tree.

Outputs, next to this file (git-ignored, shipped to the GPU box with the tree):
  fa_kernels.hsaco  gfx950 code object with every kernel (hipcc --genco)
  libfa_hip.so      C ABI of include/fa_hip.h over the HIP runtime

Run as ``python flash-attention-cpu_amd/build.py`` or via
``__graft_entry__.build()``.  Needs only hipcc / amdclang++ from /opt/rocm;
cross-compiles for gfx950 without a GPU.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HSACO = os.path.join(HERE, "fa_kernels.hsaco")
LIB = os.path.join(HERE, "libfa_hip.so")
BUILD = os.path.join(HERE, "_build")   # intermediate objects (git-ignored)

# -packed-fp32-ops: keep the compiler from emitting v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_kernels() -> str:
    _run([os.path.join(ROCM, "bin", "hipcc"), *HIP_FLAGS, "--genco",
          os.path.join(CSRC, "fa_kernels.hip"), "-o", HSACO])
    return HSACO


def build_host() -> str:
    """libfa_hip.so: fa_host.cpp (host-only C++) plus fa_scratch.hip, whose
    object carries the device-global scratch array of the allocation-free
    entry point in an embedded gfx950 code object."""
    os.makedirs(BUILD, exist_ok=True)
    scratch_obj = os.path.join(BUILD, "fa_scratch.o")
    _run([os.path.join(ROCM, "bin", "hipcc"), *HIP_FLAGS, "-fPIC", "-Wall", "-Wextra", "-c",
          os.path.join(CSRC, "fa_scratch.hip"), "-o", scratch_obj])
    _run([os.path.join(ROCM, "llvm", "bin", "clang++"), "-D__HIP_PLATFORM_AMD__",
          "-I", os.path.join(ROCM, "include"), "-fPIC", "-shared", "-O2", "-std=c++17",
          "-Wall", "-Wextra", os.path.join(CSRC, "fa_host.cpp"), scratch_obj,
          "-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-Wl,-rpath," + os.path.join(ROCM, "lib"),
          "-o", LIB])
    return LIB


def build() -> None:
    build_kernels()
    build_host()


if __name__ == "__main__":
    build()
    sys.exit(0)
