"""Builds ``libgswarp_hip.so`` (the gfx950 kernels and their C ABI) in-tree.

The library is compiled with hipcc for gfx950 only.  Floating-point flags are
part of the numerical contract: no FMA contraction, correctly rounded fp32
division and square root, and IEEE denormals, so that integer-producing
decisions (radii, tile coverage, alpha cut-offs) are reproducible by a host
compiler evaluating the same expressions.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC_DIR = PACKAGE_DIR / "csrc"
LIB_NAME = "libgswarp_hip.so"
LIB_PATH = PACKAGE_DIR / LIB_NAME
SOURCES = ("preprocess.hip", "binning.hip", "buckets.hip", "sort.hip", "render.hip", "backward.hip")
OFFLOAD_ARCH = "gfx950"

HIPCC_FLAGS = (
    "-O3",
    "-std=c++17",
    f"--offload-arch={OFFLOAD_ARCH}",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-munsafe-fp-atomics",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
)


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the gfx950 kernels cannot be built")
    return path


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source to an object and link the shared library."""
    obj_dir = PACKAGE_DIR / "_build"
    obj_dir.mkdir(exist_ok=True)
    compiler = hipcc()
    objects = []
    procs = []
    for name in SOURCES:
        src = CSRC_DIR / name
        obj = obj_dir / (name + ".o")
        objects.append(obj)
        cmd = [compiler, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((name, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = []
    for name, proc in procs:
        out, _ = proc.communicate()
        if out and (verbose or proc.returncode != 0):
            print(out, file=sys.stderr)
        if proc.returncode != 0:
            failed.append(name)
    if failed:
        raise RuntimeError(f"hipcc failed for {', '.join(failed)}")
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [compiler, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(LIB_PATH)
