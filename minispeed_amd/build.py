"""Build the native parts in-tree.

    python -m minispeed_amd.build [--verbose]

* ``libminispeed_boundary.so``: the HIP kernels for gfx950 behind a plain C
  ABI (no torch headers), compiled with hipcc;
* ``_walk.so``: a small host-only Python extension (g++, torch and pybind11
  headers) that collects the device addresses of parameter gradients and
  storages for the segment tables.

Both are written next to this file so that they travel with the source tree.
(bench.py's streaming probes are built by ``bench_probes/build.py``.)
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from typing import List

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
SOURCES = [os.path.join(PKG_DIR, "csrc", "boundary.hip")]
INCLUDE = os.path.join(REPO_DIR, "include")
OUTPUT = os.path.join(PKG_DIR, "libminispeed_boundary.so")
ARCH = "gfx950"

# -ffp-contract=off: every a*b+c the kernels do not write as fmaf stays two
#   roundings, matching the op-by-op rounding of the torch sequence they
#   replace.
# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def command(output: str = OUTPUT) -> List[str]:
    return [hipcc(), *HIP_FLAGS, f"-I{INCLUDE}", *SOURCES, "-o", output]


def build(verbose: bool = False) -> str:
    """Compile the library (always, even when an older build exists)."""
    tmp = OUTPUT + ".tmp"
    cmd = command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is
    # expected and harmless.
    noise = ("packed-fp32-ops", "--hip-link")
    log = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines()
        if line.strip() and not any(n in line for n in noise)
    )
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{log}")
    if verbose and log:
        print(log)
    os.replace(tmp, OUTPUT)
    return OUTPUT


WALK_SOURCE = os.path.join(PKG_DIR, "csrc", "walk.cpp")
WALK_OUTPUT = os.path.join(PKG_DIR, "_walk.so")


def walk_command(output: str = WALK_OUTPUT) -> List[str]:
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [sysconfig.get_paths()["include"], *cpp_extension.include_paths()]
    libdir = cpp_extension.library_paths()[0]
    return [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
            f"-D_GLIBCXX_USE_CXX11_ABI={abi}", *[f"-I{d}" for d in incs], WALK_SOURCE,
            "-o", output, f"-L{libdir}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python"]


def build_walk(verbose: bool = False) -> str:
    """Compile ``_walk.so`` (always)."""
    tmp = WALK_OUTPUT + ".tmp"
    cmd = walk_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"g++ failed ({proc.returncode}):\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, WALK_OUTPUT)
    return WALK_OUTPUT


def build_all(verbose: bool = False) -> List[str]:
    return [build(verbose=verbose), build_walk(verbose=verbose)]


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args(argv)
    for path in build_all(verbose=args.verbose):
        print(path)
    return 0


if __name__ == "__main__":
    sys.exit(main())
