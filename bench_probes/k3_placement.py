"""K3 (``ms_fused_adamw``) over one flat range with the fp32 masters and
moments placed in a chosen way: the measurement behind the state arena.

    python -m bench_probes.k3_placement {arena,separate,packed} [--elements N]
                                        [--warmup W] [--reps R]

* ``arena``: the engine's default placement (``flat.place_state`` with the
  automatic window, 36 GiB: three windows of one 108 GiB allocation, the
  gaps handed back to torch's allocator);
* ``separate``: three allocations (``place_state`` with window 0);
* ``packed``: one allocation holding the three arrays back to back.

The fp16 gradient and model copy are separate allocations, as autograd and
the module leave them.  Prints one line per placement with the mean launch
time from HIP events on the launch stream; under ``rocprofv3 --pmc`` the
same launches give the counters of each placement.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(HERE)
if REPO_DIR not in sys.path:
    sys.path.insert(0, REPO_DIR)

GPT_13B = 1_315_723_264


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("placement", choices=("arena", "separate", "packed"))
    ap.add_argument("--elements", type=int, default=GPT_13B)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--reps", type=int, default=10)
    args = ap.parse_args(argv)

    import torch

    from minispeed_amd import _native
    from minispeed_amd.boundary import LaunchTimer, adamw_params
    from minispeed_amd.flat import AUTO_SPACING, place_state

    n = args.elements
    if n <= 0 or n % 512:
        raise SystemExit("--elements must be a positive multiple of 512")
    dev = torch.device("cuda", 0)
    lib = _native.load()
    stream = _native.stream_handle(dev)
    if args.placement == "packed":
        whole = torch.zeros(3 * n, dtype=torch.float32, device=dev)
        state = [whole[k * n:(k + 1) * n] for k in range(3)]
        placement = {"bytes": 12 * n}
    else:
        bufs, where = place_state([[n, n, n]], dev, AUTO_SPACING if args.placement == "arena" else 0)
        state = bufs[0]
        placement = {"window": where.window, "arena_bytes": where.arena_bytes,
                     "held_bytes": where.held_bytes, "returned_bytes": where.returned_bytes}
    g = torch.full((n,), 0.5, dtype=torch.float16, device=dev)
    model = torch.empty(n, dtype=torch.float16, device=dev)
    table = torch.tensor([[0, n, g.data_ptr(), model.data_ptr()]], dtype=torch.int64, device=dev)
    hp = adamw_params(1e-3, (0.9, 0.999), 1e-8, 0.01, 10)
    scalars = torch.zeros(_native.SCALARS_BYTES, dtype=torch.uint8, device=dev)   # no skip, no clip
    timer = LaunchTimer(reserve=2 * args.reps)

    def k3():
        _native.check(lib.ms_fused_adamw(state[0].data_ptr(), state[1].data_ptr(), state[2].data_ptr(),
                                         None, table.data_ptr(), 1, _native.DTYPE_F16, _native.DTYPE_F16,
                                         0, n, ctypes.byref(hp), scalars.data_ptr(), stream),
                      "ms_fused_adamw")

    for _ in range(args.warmup):
        k3()
    for _ in range(args.reps):
        token = timer.start("k3")
        k3()
        timer.stop(token)
    torch.cuda.synchronize()
    ms = timer.durations_ms("k3")
    mean = sum(ms) / len(ms)
    print(json.dumps({"placement": args.placement, "elements": n, "k3_ms_mean": round(mean, 4),
                      "k3_ms_min": round(min(ms), 4), "gbps": round(28 * n / (mean * 1e-3) / 1e9, 1),
                      "state": placement}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
