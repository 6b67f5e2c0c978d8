"""Build the native library in-tree: camelid_amd/_lib/libcamelid_hip.so.

HIP sources are compiled by hipcc for gfx950 only; host-only C++ (the seam and the
synthetic-weight generator) by g++.  Every translation unit uses -ffp-contract=off:
the f32 arithmetic must match Camelid's CPU path operation for operation.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB_DIR = PKG / "_lib"
BUILD_DIR = PKG / "_build"
LIB = LIB_DIR / "libcamelid_hip.so"

HIP_SOURCES = ["engine.hip"]
HOST_SOURCES = ["seam.cpp", "synth.cpp", "gguf.cpp"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-gpu-rdc",
    "-Wall",
    "-Wno-unused-result",
    # packed FP32 (v_pk_*_f32) code generation is disabled for every HIP object
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # matrix-core results in VGPRs (the GEMM folds them with VALU code right away)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]
GXX_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-pthread", "-Wall"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the HIP backend)")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout[-4000:] + proc.stderr[-8000:])
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd[:6])} ...")


STAMPS_LIB = LIB_DIR / "libcamelid_hip_stamps.so"


def build(verbose: bool = False, stamps: bool = False) -> Path:
    """Compile every source and link the shared library; returns its path.  stamps: the
    measurement build instead (-DCM_STAMPS: the decode attention also records phase
    timestamps), linked as libcamelid_hip_stamps.so beside the product library."""
    BUILD_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    hipcc = _hipcc()
    objs: list[str] = []
    for src in HIP_SOURCES:
        obj = BUILD_DIR / (Path(src).stem + (".stamps" if stamps else "") + ".hip.o")
        _run([hipcc, *HIPCC_FLAGS, *(["-DCM_STAMPS"] if stamps else []), "-I", str(CSRC), "-c", str(CSRC / src),
              "-o", str(obj)])
        objs.append(str(obj))
    for src in HOST_SOURCES:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        _run(["g++", *GXX_FLAGS, "-I", str(CSRC), "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(str(obj))
    out = STAMPS_LIB if stamps else LIB
    tmp = out.with_suffix(".so.tmp")
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-pthread", *objs, "-o", str(tmp)])
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True, stamps="--stamps" in sys.argv[1:])
