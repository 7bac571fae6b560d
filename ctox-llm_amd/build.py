"""Builds the gfx950 code object and the C-ABI shared library in-tree.

    python ctox-llm_amd/build.py

Outputs (git-ignored, shipped with the tree):
  ctox-llm_amd/lib/ctox_kernels.hsaco  -- every HIP kernel, gfx950 only
  ctox-llm_amd/lib/libctox_hip.so      -- include/ctox_hip.h, code object embedded
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB = os.path.join(PKG, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

# Packed-FP32 instructions are kept out of every code object on this pool.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs (no accumulation-register round trips in the epilogues).
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout)
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}")


def build_kernels() -> str:
    os.makedirs(LIB, exist_ok=True)
    out = os.path.join(LIB, "ctox_kernels.hsaco")
    src = os.path.join(PKG, "csrc", "kernels", "ctox_kernels.hip")
    _run([HIPCC, *HIP_FLAGS, "--genco", src, "-o", out])
    return out


def build_noalloc() -> str:
    """The static device scratch of the allocation-free entry point: a HIP
    source compiled with hipcc (its __device__ array is registered with the
    runtime when the library loads)."""
    out = os.path.join(LIB, "noalloc.o")
    src = os.path.join(PKG, "csrc", "shim", "noalloc.hip")
    _run([HIPCC, *HIP_FLAGS, "-fPIC", "-c", f"-I{os.path.join(ROOT, 'include')}", src, "-o", out])
    return out


def build_shim(hsaco: str) -> str:
    out = os.path.join(LIB, "libctox_hip.so")
    src = os.path.join(PKG, "csrc", "shim", "ctox_hip.cpp")
    engine = os.path.join(PKG, "csrc", "shim", "engine.cpp")
    noalloc = build_noalloc()
    _run([
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
        "-D__HIP_PLATFORM_AMD__", f"-DCTOX_HSACO_PATH=\"{hsaco}\"",
        f"-I{os.path.join(ROOT, 'include')}", f"-I{os.path.join(ROCM, 'include')}",
        src, engine, noalloc, "-o", out,
        f"-L{os.path.join(ROCM, 'lib')}", "-lamdhip64", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}",
    ])
    return out


def build_all() -> None:
    hsaco = build_kernels()
    build_shim(hsaco)


if __name__ == "__main__":
    build_all()
    print("built", LIB)
