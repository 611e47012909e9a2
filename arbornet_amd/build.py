"""Build the native libraries of arbornet_amd in-tree.

* ``libarbor_hip.so``   -- the gfx950 HIP sampling library (C ABI in include/arbor_sampling.h)
* ``libarbor_synth.so`` -- seeded synthetic workloads (plain C, host only)

Both land next to this file so that they travel with the source tree. ``python -m
arbornet_amd.build`` rebuilds them.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
HIP_LIB = PKG / "libarbor_hip.so"
SYNTH_LIB = PKG / "libarbor_synth.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
OFFLOAD_ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # one rounding per fp32 operation, as the sampling contract specifies
    "-ffp-contract=off",
    # no packed-fp32 VALU instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}")


def build_hip() -> Path:
    tmp = HIP_LIB.with_suffix(".so.tmp")
    _run([HIPCC, *HIP_FLAGS, f"-I{ROOT / 'include'}", str(CSRC / "sampling.hip"), "-o", str(tmp)])
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def build_synth() -> Path:
    tmp = SYNTH_LIB.with_suffix(".so.tmp")
    _run(["gcc", "-O2", "-fPIC", "-shared", "-std=c11", "-ffp-contract=off", "-fno-fast-math",
          str(CSRC / "synth.c"), "-o", str(tmp), "-lm"])
    os.replace(tmp, SYNTH_LIB)
    return SYNTH_LIB


def build_all() -> None:
    build_synth()
    build_hip()


if __name__ == "__main__":
    build_all()
    print(f"built {HIP_LIB} and {SYNTH_LIB}")
