"""ms_boundary_scalars_noalloc against the entry points it stands for.

The no-allocation entry point runs K1 and the fold over every group with its
tile and partial slots in the library's static scratch array, then K2.  Its result must equal, bit
for bit, ms_grad_stats per group into a caller workspace followed by
ms_norm_clip, on two calls in a row, the second with a smaller input (the
scratch keeps the first call's contents).  Groups are ragged fp16 / bf16 /
fp32 gradient lists with padding rows, missing gradients, misaligned
storage and an owned range shorter than the scanned one.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from minispeed_amd import _native
from minispeed_amd.flat import FlatLayout, check_table

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
TORCH = {_native.DTYPE_F16: torch.float16, _native.DTYPE_BF16: torch.bfloat16,
         _native.DTYPE_F32: torch.float32}


def _group(rng, numels, dtype, world, rank, inject=None):
    """Ragged gradients of one group, its device segment table and the
    ms_group_scan_t fields; ``inject`` puts an inf at that flat index."""
    lay = FlatLayout(numels, rank=rank, world_size=world, zero_stage=2)
    grads, stores = [], []
    for k, n in enumerate(numels):
        if k % 5 == 3:                                   # a parameter without a gradient
            stores.append(None)
            continue
        g = torch.from_numpy(rng.standard_normal(n + 1).astype(np.float32) * 300.0).to(TORCH[dtype])
        g = g.to(DEV)[1:] if k % 4 == 1 else g.to(DEV)[:n]   # every fourth one misaligned
        if inject is not None and lay.offsets[k] <= inject < lay.offsets[k] + n:
            g[inject - lay.offsets[k]] = float("inf")
        grads.append(g)
        stores.append((g.data_ptr(), (lay.offsets[k], lay.offsets[k] + n), g.element_size()))
    table = lay.segments(0, lay.numel_padded, stores, [None] * len(numels))
    check_table(table, 0, lay.numel_padded)
    dev_table = torch.from_numpy(table).to(DEV)
    scan = _native.GroupScan(dev_table.data_ptr(), len(table), dtype, 0, lay.numel_padded,
                             lay.shard_start, lay.shard_end)
    return scan, (grads, dev_table)


def _with_workspace(lib, scans, stream, **kw):
    nb = _native.stats_blocks()
    psum = torch.empty(len(scans) * nb, dtype=torch.float64, device=DEV)
    pflag = torch.empty(len(scans) * nb, dtype=torch.int32, device=DEV)
    for g, s in enumerate(scans):
        nt = _native.scan_tiles(s.end - s.begin)
        tsum = torch.empty(max(1, nt), dtype=torch.float64, device=DEV)
        tflag = torch.empty(max(1, nt), dtype=torch.int32, device=DEV)
        _native.check(lib.ms_grad_stats(s.segs, s.nseg, s.grad_dtype, s.begin, s.end, s.own_begin,
                                        s.own_end, kw["unscale"], kw["grad_scale"], None,
                                        tsum.data_ptr(), tflag.data_ptr(), nt,
                                        psum.data_ptr() + 8 * g * nb, pflag.data_ptr() + 4 * g * nb,
                                        nb, stream), "ms_grad_stats")
    out = torch.empty(_native.SCALARS_BYTES, dtype=torch.uint8, device=DEV)
    _native.check(lib.ms_norm_clip(psum.data_ptr(), pflag.data_ptr(), nb, len(scans), 1, 1.0, 1,
                                   kw["scale"], 3, 1, 1000, 1.0, 2.0 ** 24, out.data_ptr(), None,
                                   stream), "ms_norm_clip")
    return out


def _no_alloc(lib, scans, stream, **kw):
    arr = (_native.GroupScan * max(1, len(scans)))(*scans)
    out = torch.empty(_native.SCALARS_BYTES, dtype=torch.uint8, device=DEV)
    host = torch.zeros(_native.SCALARS_BYTES, dtype=torch.uint8, pin_memory=True)
    rc = lib.ms_boundary_scalars_noalloc(arr, len(scans), kw["unscale"], kw["grad_scale"], 1, 1.0, 1,
                                         kw["scale"], 3, 1, 1000, 1.0, 2.0 ** 24, out.data_ptr(),
                                         host.data_ptr(), stream)
    _native.check(rc, "ms_boundary_scalars_noalloc")
    return out, host


def test_no_alloc_scalars_equal_the_workspace_entry_points_on_two_calls():
    lib = _native.load()
    stream = _native.stream_handle(DEV)
    rng = np.random.default_rng(21)
    kw = {"unscale": _native.SCALE_DIVIDE, "grad_scale": 1024.0, "scale": 1024.0}
    calls = [
        # (numels per group, dtype per group, world, rank, injected inf per group)
        ([[3_000_000, 7, 65_536, 1, 4099, 2_000_003], [131_072, 333, 5], [999_999]],
         [_native.DTYPE_F16, _native.DTYPE_BF16, _native.DTYPE_F32], 4, 1, [None, None, None]),
        ([[70_001, 12], [9]], [_native.DTYPE_F16, _native.DTYPE_F16], 1, 0, [None, 3]),
    ]
    for call, (sizes, dtypes, world, rank, injects) in enumerate(calls):
        print(f"[no-alloc] call {call}: {len(sizes)} groups, {sum(map(sum, sizes)):,} elements",
              flush=True)
        made = [_group(rng, s, d, world, rank, inj) for s, d, inj in zip(sizes, dtypes, injects)]
        scans = [m[0] for m in made]
        want = _with_workspace(lib, scans, stream, **kw)
        got, host = _no_alloc(lib, scans, stream, **kw)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), want.cpu()), call
        res = _native.StepScalars.from_buffer_copy(host.numpy().tobytes())
        dev = _native.StepScalars.from_buffer_copy(want.cpu().numpy().tobytes())
        assert res.ready == 1 and dev.ready == 0, call     # the host copy's ready word
        dev.ready = 1
        assert bytes(res) == bytes(dev), call
        assert res.overflow == (1 if any(i is not None for i in injects) else 0)
        if not res.overflow:
            assert res.sumsq > 0 and res.norm > 1.0 and res.clip_applied == 1


def test_no_alloc_refuses_more_groups_than_its_scratch():
    lib = _native.load()
    n = _native.SCRATCH_MAX_GROUPS + 1
    arr = (_native.GroupScan * n)()
    out = torch.empty(_native.SCALARS_BYTES, dtype=torch.uint8, device=DEV)
    rc = lib.ms_boundary_scalars_noalloc(arr, n, 0, 1.0, 0, 0.0, 0, 1.0, 0, 0, 1, 1.0, 1.0,
                                         out.data_ptr(), None, _native.stream_handle(DEV))
    assert rc == _native.ESCRATCH
    assert b"MS_SCRATCH_MAX_GROUPS" in lib.ms_error_string(rc)
