"""Ahead-of-time build of libpcdevice_hip.so for gfx950 (no JIT, no cache outside the tree).

The library is one host translation unit (csrc/pcdevice.hip) plus one unit per
(operand type, GEMM tile) instantiation of the phase kernels
(csrc/phase_inst.hip compiled with -DPCD_OP_ID/-DPCD_BM/-DPCD_BN); the units
compile in parallel and link into one shared object.
"""
from __future__ import annotations

import os
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libpcdevice_hip.so")
HOST_SOURCE = os.path.join(CSRC, "pcdevice.hip")
INST_SOURCE = os.path.join(CSRC, "phase_inst.hip")

OPS = {"f32": 0, "bf16": 1, "f16": 2}
TILES = [(32, 32), (64, 64), (64, 128), (64, 256), (128, 128), (256, 128), (256, 256)]

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # no packed-fp32 instructions: some of their forms have misbehaved on this pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]


def _units():
    """(source, extra flags, object name) of every translation unit."""
    units = [(HOST_SOURCE, [], "pcdevice.o")]
    for op, op_id in OPS.items():
        for bm, bn in TILES:
            units.append((INST_SOURCE, [f"-DPCD_OP_ID={op_id}", f"-DPCD_BM={bm}", f"-DPCD_BN={bn}"],
                          f"phase_{op}_{bm}x{bn}.o"))
    units.extend(_direct_units())
    return units


def _direct_units():
    """The direct-weight 64 x 128 tile of the 16-bit operand types."""
    return [(INST_SOURCE, [f"-DPCD_OP_ID={OPS[op]}", "-DPCD_BM=64", "-DPCD_BN=128", "-DPCD_WD=1"],
             f"phase_{op}_64x128d.o") for op in ("bf16", "f16")]


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in l)
    return res.returncode, out


def build_library(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile the HIP library in-tree (always recompiles every unit)."""
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    jobs = jobs or min(8, os.cpu_count() or 1)
    with tempfile.TemporaryDirectory(prefix="pcd_build_") as tmpdir:
        units = _units()
        cmds = [[hipcc, *HIPCC_FLAGS, *flags, "-c", src, "-o", os.path.join(tmpdir, obj)]
                for src, flags, obj in units]
        with ThreadPoolExecutor(jobs) as ex:
            results = list(ex.map(_run, cmds))
        for (src, flags, obj), (rc, out) in zip(units, results):
            if rc != 0:
                raise RuntimeError(f"hipcc failed on {obj} ({rc}):\n{out}")
            if verbose and out.strip():
                print(out)
        check_direct_asm(hipcc, tmpdir, jobs)
        tmp = LIB + ".tmp"
        # -z defs: a tile the host dispatches but no unit instantiates fails here,
        # not when the library is loaded
        rc, out = _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,-z,defs",
                        *[os.path.join(tmpdir, obj) for _, _, obj in units], "-o", tmp])
        if rc != 0:
            raise RuntimeError(f"link failed ({rc}):\n{out}")
    os.replace(tmp, LIB)
    return LIB


def check_direct_asm(hipcc: str, tmpdir: str, jobs: int) -> None:
    """Compile the direct-weight units to device assembly and check their inline-asm loads' waits."""
    from predicitivecoding_amd.asm_check import check_asm

    units = _direct_units()
    cmds = [[hipcc, *HIPCC_FLAGS, *flags, "--offload-device-only", "-S", src,
             "-o", os.path.join(tmpdir, obj.replace(".o", ".s"))] for src, flags, obj in units]
    with ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(_run, cmds))
    for (src, flags, obj), (rc, out) in zip(units, results):
        if rc != 0:
            raise RuntimeError(f"hipcc -S failed on {obj} ({rc}):\n{out}")
        with open(os.path.join(tmpdir, obj.replace(".o", ".s"))) as f:
            found = check_asm(f.read())
        if not found:
            raise RuntimeError(f"{obj}: no phase kernel in the device assembly")
        bad = {k: v for k, v in found.items() if v}
        if bad:
            lines = [f"  {k}: {v[0]} (+{len(v) - 1} more)" for k, v in bad.items()]
            raise RuntimeError(f"{obj}: inline-asm loads read or overwritten in flight:\n" + "\n".join(lines))


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
