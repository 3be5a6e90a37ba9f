"""Build step of colizig_amd: compiles the HIP library for gfx950 and the
host loader, in-tree (the built .so files sit next to this file).

    python -m colizig_amd.build
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
HIP_LIB = os.path.join(HERE, "libcolizig_hip.so")
LOADER_LIB = os.path.join(HERE, "libcolizig_gpu.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-shared",
    "-std=c++17",
    # every fused multiply-add is written out; nothing is contracted
    "-ffp-contract=off",
    # no packed-FP32 instructions in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build_hip() -> str:
    tmp = HIP_LIB + ".tmp"
    _run([HIPCC, *HIP_FLAGS, "-I", os.path.join(ROOT, "include"), "-o", tmp,
          os.path.join(CSRC, "colizig_hip.hip")])
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def build_loader() -> str:
    tmp = LOADER_LIB + ".tmp"
    _run(["g++", "-O2", "-fPIC", "-shared", "-std=c++17", "-Wall", "-o", tmp,
          os.path.join(CSRC, "host", "cz_gpu_loader.cpp"), "-ldl"])
    os.replace(tmp, LOADER_LIB)
    return LOADER_LIB


def build_all() -> None:
    build_hip()
    build_loader()


if __name__ == "__main__":
    build_all()
    print("built", HIP_LIB, LOADER_LIB)
