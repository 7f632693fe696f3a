"""Builds ``heimdall_amd/libbifrost_hip.so`` from ``heimdall_amd/csrc/*.hip`` with hipcc for gfx950.

    python -m heimdall_amd.build          # or heimdall_amd.build.build_library()

Every source is compiled to its own object (in parallel, under ``heimdall_amd/_build/``) and the objects are linked
into one shared library. Kernels never call device code of another source file, so no relocatable device code is
needed. The library is built in-tree (next to this file) so that it travels with the source tree.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libbifrost_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # no packed fp32 VALU ops in device code (v_pk_fma_f32 and friends)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]
NOISE = "'-packed-fp32-ops' is not a recognized feature"      # the host pass does not know the device feature


def sources():
    return sorted(CSRC.glob("*.hip"))


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in res.stderr.splitlines() if NOISE not in l)
    if res.returncode != 0:
        raise subprocess.CalledProcessError(res.returncode, cmd, res.stdout, err)
    return err


def build_library(verbose: bool = False, jobs: int = 0) -> Path:
    """Compile every HIP source and link the shared library; raises CalledProcessError on a compile error."""
    OBJ.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    cmds = [[HIPCC, *FLAGS, "-c", str(s), "-o", str(OBJ / (s.stem + ".o"))] for s in srcs]
    if verbose:
        for c in cmds:
            print(" ".join(c), flush=True)
    with ThreadPoolExecutor(jobs) as ex:
        errs = list(ex.map(_run, cmds))
    tmp = LIB.with_suffix(".so.tmp")
    link = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
            *(str(OBJ / (s.stem + ".o")) for s in srcs)]
    if verbose:
        print(" ".join(link), flush=True)
    errs.append(_run(link))
    if verbose:
        for e in errs:
            if e.strip():
                print(e, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build_library(verbose=True))
