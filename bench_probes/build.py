"""Build ``libms_hbm_probe.so`` in-tree (the streaming probes behind
``bench.py --hbm-ceilings``).

    python -m bench_probes.build [--verbose]

Same hipcc flags as the boundary library (minispeed_amd/build.py), so a
probe and the kernel it is compared with are compiled alike.
"""

from __future__ import annotations

import argparse
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(HERE)
if REPO_DIR not in sys.path:
    sys.path.insert(0, REPO_DIR)

from minispeed_amd.build import HIP_FLAGS, hipcc  # noqa: E402

PROBE_SOURCE = os.path.join(HERE, "hbm_probe.hip")
PROBE_OUTPUT = os.path.join(HERE, "libms_hbm_probe.so")


def build_probe(verbose: bool = False) -> str:
    """Compile ``libms_hbm_probe.so`` (always)."""
    tmp = PROBE_OUTPUT + ".tmp"
    cmd = [hipcc(), *HIP_FLAGS, f"-I{HERE}", PROBE_SOURCE, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, PROBE_OUTPUT)
    return PROBE_OUTPUT


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args(argv)
    print(build_probe(verbose=args.verbose))
    return 0


if __name__ == "__main__":
    sys.exit(main())
