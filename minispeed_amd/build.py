"""Build ``libminispeed_boundary.so`` in-tree with hipcc for gfx950.

    python -m minispeed_amd.build [--verbose]

The library is a plain C-ABI shared object (no torch headers); it is written
next to this file so that it travels with the source tree.
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


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args(argv)
    path = build(verbose=args.verbose)
    print(path)
    return 0


if __name__ == "__main__":
    sys.exit(main())
