"""Ahead-of-time build of libpcdevice_hip.so for gfx950 (no JIT, no cache outside the tree)."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libpcdevice_hip.so")
SOURCES = [os.path.join(HERE, "csrc", "pcdevice.hip")]
DEPENDS = SOURCES + [os.path.join(HERE, "csrc", "pc_kernels.hpp"), os.path.join(ROOT, "include", "pcdevice.h")]

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # no packed-fp32 instructions: some of their forms have misbehaved on this pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]


def build_library(verbose: bool = False) -> str:
    """Compile the HIP library in-tree (always recompiles)."""
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = LIB + ".tmp"
    cmd = [hipcc, *HIPCC_FLAGS, *SOURCES, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{out}")
    if verbose and out.strip():
        print(out)
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> str | None:
    """Compile the CPU oracle (test infrastructure) with its Makefile."""
    oracle_dir = os.path.join(ROOT, "oracle")
    if not os.path.isdir(oracle_dir):
        return None
    subprocess.run(["make", "-s", "-B", "-C", oracle_dir], check=True)
    return os.path.join(oracle_dir, "libpcoracle.so")


if __name__ == "__main__":
    print(build_library(verbose=True))
    print(build_oracle())
