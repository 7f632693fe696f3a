"""Builds ``heimdall_amd/libbifrost_hip.so`` from ``heimdall_amd/csrc/*.hip`` with hipcc for gfx950.

    python -m heimdall_amd.build          # or heimdall_amd.build.build_library()

The library is built in-tree (next to this file) so that it travels with the source tree.
"""
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libbifrost_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-shared", "-fPIC",
    # no packed fp32 VALU ops in device code (v_pk_fma_f32 and friends)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def sources():
    return sorted(str(p) for p in CSRC.glob("*.hip"))


def build_library(verbose: bool = False) -> Path:
    """Compile every HIP source into one shared library; raises CalledProcessError on a compile error."""
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, "-o", str(tmp), *sources()]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"    # host pass does not know the device feature
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise subprocess.CalledProcessError(res.returncode, cmd, res.stdout, err)
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build_library(verbose=True))
