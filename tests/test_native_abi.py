"""The C-ABI library on the CPU: it loads, exports exactly what
include/minispeed_boundary.h declares, its structs have the header's layout,
and host-side argument errors come back as codes before anything launches.
No kernel is launched here."""

from __future__ import annotations

import ctypes
import os
import re
import shutil
import subprocess

import pytest

from minispeed_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "minispeed_boundary.h")


def _declared_functions():
    text = open(HEADER, encoding="utf-8").read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ms_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_with_matching_abi():
    lib = _native.load()
    assert lib.ms_abi_version() == _native.ABI_VERSION
    assert _native.stats_blocks() >= 256


def test_every_declared_symbol_is_exported_and_typed():
    declared = _declared_functions()
    assert "ms_fused_adamw" in declared and len(declared) >= 7
    lib = ctypes.CDLL(_native.library_path())
    for name in declared:
        assert hasattr(lib, name), name
        assert name in _native.SIGNATURES, name
    assert set(_native.SIGNATURES) == set(declared)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_struct_layout_matches_header(tmp_path):
    src = tmp_path / "probe.c"
    src.write_text(r'''
#include <stddef.h>
#include <stdio.h>
#include "minispeed_boundary.h"
#define F(T, m) printf(#T "." #m " %zu\n", offsetof(T, m));
int main(void) {
  printf("ms_segment_t %zu\n", sizeof(ms_segment_t));
  F(ms_segment_t, begin) F(ms_segment_t, numel) F(ms_segment_t, grad) F(ms_segment_t, model)
  printf("ms_step_scalars_t %zu\n", sizeof(ms_step_scalars_t));
  F(ms_step_scalars_t, overflow) F(ms_step_scalars_t, clip_applied) F(ms_step_scalars_t, sumsq)
  F(ms_step_scalars_t, norm) F(ms_step_scalars_t, coef) F(ms_step_scalars_t, coef64)
  F(ms_step_scalars_t, next_scale) F(ms_step_scalars_t, next_good_steps)
  F(ms_step_scalars_t, next_skipped_steps)
  printf("ms_adamw_params_t %zu\n", sizeof(ms_adamw_params_t));
  F(ms_adamw_params_t, neg_lr) F(ms_adamw_params_t, bias_c2) F(ms_adamw_params_t, grad_scale)
  F(ms_adamw_params_t, decay) F(ms_adamw_params_t, unscale)
  printf("ms_group_scan_t %zu\n", sizeof(ms_group_scan_t));
  F(ms_group_scan_t, segs) F(ms_group_scan_t, nseg) F(ms_group_scan_t, grad_dtype)
  F(ms_group_scan_t, begin) F(ms_group_scan_t, end) F(ms_group_scan_t, own_begin)
  F(ms_group_scan_t, own_end)
  printf("ms_accum_row_t %zu\n", sizeof(ms_accum_row_t));
  F(ms_accum_row_t, dst) F(ms_accum_row_t, src) F(ms_accum_row_t, numel) F(ms_accum_row_t, first)
  F(ms_accum_row_t, reserved) F(ms_accum_row_t, tile_sumsq) F(ms_accum_row_t, tile_flag)
  printf("MS_ACCUM_ROWS_PER_LAUNCH %d\n", MS_ACCUM_ROWS_PER_LAUNCH);
  printf("MS_ACCUM_TILE %d\n", MS_ACCUM_TILE);
  printf("MS_SCRATCH_MAX_GROUPS %d\n", MS_SCRATCH_MAX_GROUPS);
  printf("MS_SCRATCH_MAX_TILES %d\n", MS_SCRATCH_MAX_TILES);
  printf("MS_SCAN_TILE %d\n", MS_SCAN_TILE);
  printf("MS_ESCRATCH %d\n", MS_ESCRATCH);
  return 0;
}
''')
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)], check=True)
    lines = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    got = dict(line.rsplit(" ", 1) for line in lines if line)
    classes = {"ms_segment_t": _native.Segment, "ms_step_scalars_t": _native.StepScalars,
               "ms_adamw_params_t": _native.AdamWParams, "ms_group_scan_t": _native.GroupScan,
               "ms_accum_row_t": _native.AccumRow}
    assert int(got.pop("MS_ACCUM_ROWS_PER_LAUNCH")) == _native.ACCUM_ROWS_PER_LAUNCH
    assert int(got.pop("MS_ACCUM_TILE")) == _native.ACCUM_TILE
    assert int(got.pop("MS_SCRATCH_MAX_GROUPS")) == _native.SCRATCH_MAX_GROUPS
    assert int(got.pop("MS_SCRATCH_MAX_TILES")) == _native.SCRATCH_MAX_TILES
    assert int(got.pop("MS_SCAN_TILE")) == _native.SCAN_TILE
    assert int(got.pop("MS_ESCRATCH")) == _native.ESCRATCH
    for key, value in got.items():
        if "." in key:
            cname, field = key.split(".")
            assert getattr(classes[cname], field).offset == int(value), key
        else:
            assert ctypes.sizeof(classes[key]) == int(value), key


def test_host_argument_errors_return_codes_without_launching():
    lib = _native.load()
    EINVAL, ETABLE, EBLOCKS = -1, -2, -3
    nb = _native.stats_blocks()
    tile = _native.SCAN_TILE

    def k1(segs, nseg, dtype, begin, end, unscale, scale, flat, ts, tf, nt, bs, bf, nblk):
        return lib.ms_grad_stats(segs, nseg, dtype, begin, end, begin, end, unscale, scale, flat,
                                 ts, tf, nt, bs, bf, nblk, None)
    # bad dtype / negative range / missing outputs / unpaired statistics
    # pointers / small workspaces / empty table
    assert k1(None, 0, 7, 0, 10, 0, 1.0, None, 8, 8, 1, 8, 8, nb) == EINVAL
    assert k1(None, 0, 1, 10, 5, 0, 1.0, None, 8, 8, 1, 8, 8, nb) == EINVAL
    assert k1(None, 0, 1, 0, 10, 0, 1.0, None, None, None, 1, None, None, nb) == EINVAL
    assert k1(None, 0, 1, 0, 10, 0, 1.0, None, None, None, 1, 8, 8, nb) == EINVAL
    assert k1(None, 0, 1, 0, 10, 0, 1.0, None, 8, None, 1, 8, 8, nb) == EINVAL
    assert k1(None, 0, 1, 0, 10, 0, 1.0, None, 8, 8, 1, None, None, nb) == EINVAL
    assert k1(None, 0, 1, 0, 10, 0, 1.0, None, 8, 8, 1, 8, 8, nb - 1) == EBLOCKS
    assert k1(None, 0, 1, 0, 10, 0, 1.0, None, 8, 8, 0, 8, 8, nb) == EBLOCKS
    assert k1(None, 0, 1, 0, 2 * tile + 1, 0, 1.0, None, 8, 8, 2, 8, 8, nb) == EBLOCKS
    assert k1(None, 0, 1, 0, 2 * tile + 1, 0, 1.0, None, 8, 8, 3, 8, 8, nb) == ETABLE
    assert k1(None, 0, 1, 0, 10, 0, 1.0, None, 8, 8, 1, 8, 8, nb) == ETABLE
    assert k1(None, 0, 1, 0, 10, 1, 0.0, 8, None, None, 0, None, None, nb) == ETABLE
    assert lib.ms_norm_clip(None, None, nb, 1, 0, 0.0, 0, 1.0, 0, 0, 1, 1.0, 1.0, None, None,
                            None) == EINVAL
    assert lib.ms_norm_clip(8, 8, nb - 1, 1, 0, 0.0, 0, 1.0, 0, 0, 1, 1.0, 1.0, 8, None,
                            None) == EBLOCKS
    assert lib.ms_norm_clip(8, 8, nb, 1, 0, 0.0, 0, 1.0, 0, 0, 0, 1.0, 1.0, 8, None, None) == EINVAL
    hp = _native.AdamWParams()
    assert lib.ms_fused_adamw(8, 8, 8, None, None, 0, 9, 1, 0, 10, ctypes.byref(hp), 8, None) == EINVAL
    assert lib.ms_fused_adamw(8, 8, 8, None, None, 0, 1, 1, 0, 10, None, 8, None) == EINVAL
    assert lib.ms_fused_adamw(8, 8, 8, None, None, 0, 1, 1, 0, 10, ctypes.byref(hp), 8, None) == ETABLE
    assert lib.ms_fused_adamw(None, None, None, None, None, 0, 1, 1, 4, 4, ctypes.byref(hp), 8, None) == 0
    hp.unscale = 1
    hp.grad_scale = 0.0
    assert lib.ms_fused_adamw(8, 8, 8, None, 8, 1, 1, 1, 0, 10, ctypes.byref(hp), 8, None) == EINVAL
    hp.unscale = _native.SCALE_MULTIPLY           # K3 only divides
    hp.grad_scale = 2.0
    assert lib.ms_fused_adamw(8, 8, 8, None, 8, 1, 1, 1, 0, 10, ctypes.byref(hp), 8, None) == EINVAL
    # K1: scaling mode out of range; divide by a non-positive scale
    assert k1(8, 1, 0, 0, 10, 3, 1.0, 8, None, None, 0, None, None, 0) == EINVAL
    assert k1(8, 1, 0, 0, 10, _native.SCALE_DIVIDE, -1.0, 8, None, None, 0, None, None, 0) == EINVAL
    assert lib.ms_cast_to_model(None, 0, 10, 8, 1, 1, None) == EINVAL
    assert lib.ms_cast_to_model(8, 0, 10, None, 0, 1, None) == ETABLE
    assert lib.ms_cast_to_model(8, 0, 10, 8, 1, 5, None) == EINVAL
    assert lib.ms_cast_to_model(None, 3, 3, None, 0, 1, None) == 0
    # the no-allocation boundary scan: group count beyond its scratch, bad
    # arguments, and a bad group, all refused before any device call
    scans = (_native.GroupScan * 9)()
    noalloc = lib.ms_boundary_scalars_noalloc
    assert noalloc(scans, 9, 0, 1.0, 0, 0.0, 0, 1.0, 0, 0, 1, 1.0, 1.0, 8, None, None) == _native.ESCRATCH
    assert noalloc(scans, 1, 0, 1.0, 0, 0.0, 0, 1.0, 0, 0, 1, 1.0, 1.0, None, None, None) == EINVAL
    assert noalloc(None, 1, 0, 1.0, 0, 0.0, 0, 1.0, 0, 0, 1, 1.0, 1.0, 8, None, None) == EINVAL
    assert noalloc(scans, 1, 0, 1.0, 0, 0.0, 0, 1.0, 0, 0, 0, 1.0, 1.0, 8, None, None) == EINVAL
    scans[0] = _native.GroupScan(None, 0, 7, 0, 10, 0, 10)
    assert noalloc(scans, 1, 0, 1.0, 0, 0.0, 0, 1.0, 0, 0, 1, 1.0, 1.0, 8, None, None) == EINVAL
    scans[0] = _native.GroupScan(None, 0, 1, 0, 10, 0, 10)
    assert noalloc(scans, 1, 0, 1.0, 0, 0.0, 0, 1.0, 0, 0, 1, 1.0, 1.0, 8, None, None) == ETABLE
    # a group with more tiles than the scratch holds
    big = _native.SCRATCH_MAX_TILES * _native.SCAN_TILE + 1
    scans[0] = _native.GroupScan(8, 1, 1, 0, big, 0, big)
    assert noalloc(scans, 1, 0, 1.0, 0, 0.0, 0, 1.0, 0, 0, 1, 1.0, 1.0, 8, None, None) == _native.ESCRATCH
    # batched K5: dtype, row count, a NULL row array, a negative size, a
    # missing address; empty rows launch nothing
    rows = (_native.AccumRow * 3)()
    acc = lib.ms_accumulate_grads
    assert acc(rows, 3, 5, 0, 1.0, None) == EINVAL
    assert acc(rows, -1, 1, 0, 1.0, None) == EINVAL
    assert acc(None, 1, 1, 0, 1.0, None) == EINVAL
    assert acc(None, 0, 1, 0, 1.0, None) == 0
    assert acc(rows, 3, 1, 0, 1.0, None) == 0           # three rows of numel 0
    assert acc(rows, 3, 1, _native.SCALE_MULTIPLY, 2.0, None) == EINVAL   # statistics only divide
    assert acc(rows, 3, 1, _native.SCALE_DIVIDE, 0.0, None) == EINVAL
    rows[1] = _native.AccumRow(8, 8, -1, 1, 0, None, None)
    assert acc(rows, 3, 1, 0, 1.0, None) == EINVAL
    rows[1] = _native.AccumRow(None, 8, 10, 1, 0, None, None)
    assert acc(rows, 3, 1, 0, 1.0, None) == EINVAL
    rows[1] = _native.AccumRow(8, 8, 10, 1, 0, 8, None)        # slots come in pairs
    assert acc(rows, 3, 1, 0, 1.0, None) == EINVAL
    fold = lib.ms_reduce_tile_stats
    assert fold(None, None, 0, None, 8, nb, None) == EINVAL
    assert fold(None, None, 5, 8, 8, nb, None) == EINVAL
    assert fold(8, 8, -1, 8, 8, nb, None) == EINVAL
    assert fold(8, 8, 5, 8, 8, nb - 1, None) == EBLOCKS
    assert lib.ms_accumulate_grad(None, None, 1, 0, 1, None) == 0
    assert lib.ms_accumulate_grad(None, 8, 1, 10, 1, None) == EINVAL
    assert lib.ms_accumulate_grad(8, 8, 4, 10, 1, None) == EINVAL
    for code in (0, EINVAL, ETABLE, EBLOCKS, _native.ESCRATCH):
        assert lib.ms_error_string(code)
    with pytest.raises(RuntimeError, match="segment count"):
        _native.check(ETABLE, "probe")


def test_integration_stub_matches_the_binding():
    """The ctypes stub a maintainer copies from INTEGRATION.md declares every
    entry point with the binding's argument types."""
    with open(os.path.join(ROOT, "INTEGRATION.md")) as f:
        text = f.read()
    short = {"P": "P", "I32": "I32", "I64": "I64", "F": "F", "D": "D"}
    ctype = {ctypes.c_void_p: "P", ctypes.c_int32: "I32", ctypes.c_int64: "I64",
             ctypes.c_float: "F", ctypes.c_double: "D"}
    stubs = re.findall(r"lib\.(\w+)\.argtypes = \[([^\]]*)\]", text)
    assert {name for name, _ in stubs} >= {"ms_grad_stats", "ms_norm_clip", "ms_fused_adamw",
                                           "ms_cast_to_model", "ms_accumulate_grads",
                                           "ms_reduce_tile_stats"}
    for name, body in stubs:
        got = [short.get(a.strip(), "P") for a in re.split(r",\s*(?![^(]*\))", body) if a.strip()]
        want = [ctype.get(t, "P") for t in _native.SIGNATURES[name][1]]
        assert got == want, name


def test_header_constants_match_the_binding():
    with open(HEADER) as f:
        text = f.read()
    consts = {k: int(v) for k, v in re.findall(r"\b(MS_[A-Z0-9_]+)\s*=\s*(-?\d+)", text)}
    assert int(re.search(r"#define MS_ABI_VERSION (\d+)", text).group(1)) == _native.ABI_VERSION
    for name in ("DTYPE_F32", "DTYPE_F16", "DTYPE_BF16", "SCALE_NONE", "SCALE_DIVIDE", "SCALE_MULTIPLY"):
        assert consts["MS_" + name] == getattr(_native, name), name


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setenv("MINISPEED_AMD_LIB", str(tmp_path / "absent.so"))
    monkeypatch.setattr(_native, "_lib", None)
    with pytest.raises(_native.NativeLibraryError):
        _native.load()


def test_pointer_walk_extension_loads_and_defers_host_tensors():
    """The C++ walk is built in-tree and hands every tensor it does not
    accept (here: host tensors) back to the Python checks by index."""
    import numpy as np
    import torch
    from torch import nn

    from minispeed_amd import _walk

    params = [nn.Parameter(torch.zeros(3)), nn.Parameter(torch.zeros(2))]
    out = np.full(3, -7, dtype=np.int64)
    bad, keep = _walk.grad_pointers(params, np.array([3, 2], dtype=np.int64), 0, out)
    assert (bad, keep, list(out[:2])) == (-1, [None, None], [0, 0])
    params[1].grad = torch.ones(2)
    bad, keep = _walk.grad_pointers(params, np.array([3, 2], dtype=np.int64), 0, out)
    assert bad == 1 and keep == [None]
    assert _walk.model_pointers(params, 0, out) == 0
    with pytest.raises(ValueError):
        _walk.grad_pointers(params, np.array([3], dtype=np.int64), 0, out)
    # record_streams skips None and host tensors (nothing to record) and
    # refuses what is not a tensor
    assert _walk.record_streams([None, torch.zeros(2), params[0]], 1, 0, 0) == 0
    with pytest.raises(TypeError):
        _walk.record_streams([3], 1, 0, 0)


def test_probe_library_abi_and_refusals():
    """libms_hbm_probe.so (bench.py --hbm-ceilings only): its ABI version,
    every function its header declares, and bad arguments refused in host
    code before anything is launched."""
    here = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "bench_probes")
    path = os.path.join(here, "libms_hbm_probe.so")
    if not os.path.exists(path):
        pytest.skip("probe library not built (python -m bench_probes.build)")
    lib = ctypes.CDLL(path)
    header = open(os.path.join(here, "minispeed_hbm_probe.h")).read()
    version = int(re.search(r"#define MSP_ABI_VERSION (\d+)", header).group(1))
    lib.msp_abi_version.restype = ctypes.c_int
    assert lib.msp_abi_version() == version == 2
    for name in re.findall(r"^int (msp_\w+)\(", header, re.M):
        assert hasattr(lib, name), name
    P = ctypes.c_void_p
    lib.msp_adam_layout.restype = ctypes.c_int
    lib.msp_adam_layout.argtypes = [ctypes.POINTER(P), P, P, ctypes.c_int64, ctypes.c_int32,
                                    ctypes.c_int32, P]
    state = (P * 3)(16, 32, 48)
    ok = dict(state=state, g=64, copy=128, n=4096, inter=0, chunk=0)

    def call(**kw):
        a = dict(ok, **kw)
        return lib.msp_adam_layout(a["state"], a["g"], a["copy"], a["n"], a["inter"], a["chunk"],
                                   None)
    for bad in (dict(n=0), dict(n=4095), dict(inter=256), dict(inter=4096, n=2048 * 3),
                dict(chunk=-1), dict(g=None), dict(copy=66), dict(state=(P * 3)(16, 0, 48)),
                dict(state=(P * 3)(16, 40, 48))):
        assert call(**bad) == -1, bad
