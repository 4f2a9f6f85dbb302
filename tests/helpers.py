"""Shared helpers of the test suite (inputs, segment tables, C-ABI calls)."""

from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence

import numpy as np
import torch

from minispeed_amd import _native
from minispeed_amd.boundary import adamw_params
from minispeed_amd.flat import FlatLayout, check_table

DEV = "cuda"

HALF_SPECIALS = {
    torch.float16: [0x7C00, 0xFC00, 0x7E00, 0x7C01, 0xFE01, 0x7BFF, 0x0001, 0x8001, 0x03FF],
    torch.bfloat16: [0x7F80, 0xFF80, 0x7FC0, 0x7F81, 0xFFC1, 0x7F7F, 0x0001, 0x8001, 0x007F],
    torch.float32: [0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800001, 0xFFC00001, 0x7F7FFFFF,
                    0x00000001, 0x80000001, 0x007FFFFF],
}
# first five of each list are inf/nan encodings, the rest finite extremes


def gpu_available() -> bool:
    return torch.cuda.is_available()


def ragged_grads(shapes, dtype, std, seed, scale=1.0) -> List[torch.Tensor]:
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(*s, generator=g) * std * scale).to(dtype) for s in shapes]


def set_bits(t: torch.Tensor, index: int, pattern: int) -> None:
    """Write a raw bit pattern into element ``index`` of a CPU tensor."""
    flat = t.view(-1)
    if t.dtype in (torch.float16, torch.bfloat16):
        flat.view(torch.int16)[index] = np.int16(np.uint16(pattern))
    else:
        flat.view(torch.int32)[index] = np.int32(np.uint32(pattern))


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous().reshape(-1)
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().copy()
    return t.view(torch.int32).numpy().copy()


def store(t: Optional[torch.Tensor], begin: int):
    if t is None:
        return None
    return (t.data_ptr(), (begin, begin + t.numel()), t.element_size())


class Table:
    """A device segment table built from ragged device tensors."""

    def __init__(self, layout: FlatLayout, lo: int, hi: int, grads, models):
        arr = layout.segments(lo, hi, grads, models)
        check_table(arr, lo, hi)
        self.host = arr
        self.nseg = int(arr.shape[0])
        self.dev = torch.from_numpy(arr.copy()).to(DEV) if self.nseg else None

    @property
    def ptr(self):
        return self.dev.data_ptr() if self.dev is not None else None


def layout_for(numels: Sequence[int], world_size=1, rank=0, stage=0) -> FlatLayout:
    return FlatLayout(list(numels), rank=rank, world_size=world_size, zero_stage=stage)


def stream() -> int:
    return _native.stream_handle(torch.device(DEV))


def k1(table: Table, dtype: torch.dtype, begin, end, own_begin, own_end, scale=1.0,
       flat: Optional[torch.Tensor] = None, nblk: Optional[int] = None, tiles: bool = False):
    """Run ms_grad_stats with stats; return (partials fp64, flags) on CPU,
    followed with ``tiles`` by (tile sums fp64, tile flags).  The tile slots
    start as NaN / -1, plus one spare slot that must stay so."""
    lib = _native.load()
    nb = nblk or _native.stats_blocks()
    nt = _native.scan_tiles(end - begin)
    psum = torch.full((nb,), float("nan"), dtype=torch.float64, device=DEV)
    pflag = torch.full((nb,), -1, dtype=torch.int32, device=DEV)
    tsum = torch.full((nt + 1,), float("nan"), dtype=torch.float64, device=DEV)
    tflag = torch.full((nt + 1,), -1, dtype=torch.int32, device=DEV)
    rc = lib.ms_grad_stats(
        table.ptr, table.nseg, _native.ms_dtype(dtype), begin, end, own_begin, own_end,
        1 if scale != 1.0 else 0, float(np.float32(scale)),
        flat.data_ptr() if flat is not None else None, tsum.data_ptr(), tflag.data_ptr(), nt,
        psum.data_ptr(), pflag.data_ptr(), nb, stream())
    _native.check(rc, "ms_grad_stats")
    torch.cuda.synchronize()
    out = (psum.cpu().numpy(), pflag.cpu().numpy())
    if tiles:
        ts, tf = tsum.cpu().numpy(), tflag.cpu().numpy()
        assert np.isnan(ts[nt]) and tf[nt] == -1, "K1 wrote past its tile slots"
        out += (ts[:nt], tf[:nt])
    return out


def k2(psum: np.ndarray, pflag: np.ndarray, ngroups=1, has_clip=False, max_norm=0.0,
       scaler=(False, 1.0, 0, 0, 1000, 1.0, 2.0 ** 24)) -> _native.StepScalars:
    lib = _native.load()
    nb = _native.stats_blocks()
    ps = torch.from_numpy(np.ascontiguousarray(psum, dtype=np.float64)).to(DEV)
    pf = torch.from_numpy(np.ascontiguousarray(pflag, dtype=np.int32)).to(DEV)
    out = torch.zeros(_native.SCALARS_BYTES, dtype=torch.uint8, device=DEV)
    en, scale, good, skipped, window, mn, mx = scaler
    rc = lib.ms_norm_clip(ps.data_ptr(), pf.data_ptr(), nb, ngroups, 1 if has_clip else 0,
                          float(max_norm), 1 if en else 0, float(scale), int(good), int(skipped),
                          int(window), float(mn), float(mx), out.data_ptr(), None, stream())
    _native.check(rc, "ms_norm_clip")
    torch.cuda.synchronize()
    return _native.StepScalars.from_buffer_copy(out.cpu().numpy().tobytes())


def scalars_device(overflow=0, clip_applied=0, coef=1.0) -> torch.Tensor:
    s = _native.StepScalars()
    s.overflow = overflow
    s.clip_applied = clip_applied
    s.coef = float(np.float32(coef))
    s.coef64 = float(coef)
    raw = np.frombuffer(bytes(s), dtype=np.uint8).copy()
    return torch.from_numpy(raw).to(DEV)


def k3(table: Table, gdtype, mdtype, begin, end, p, m, v, hp, scalars: torch.Tensor,
       flat_grad: Optional[torch.Tensor] = None):
    lib = _native.load()
    rc = lib.ms_fused_adamw(p.data_ptr(), m.data_ptr(), v.data_ptr(),
                            flat_grad.data_ptr() if flat_grad is not None else None,
                            table.ptr, table.nseg, _native.ms_dtype(gdtype), _native.ms_dtype(mdtype),
                            begin, end, ctypes.byref(hp), scalars.data_ptr(), stream())
    _native.check(rc, "ms_fused_adamw")
    torch.cuda.synchronize()


def k4(table: Table, mdtype, flat: torch.Tensor, begin, end):
    lib = _native.load()
    rc = lib.ms_cast_to_model(flat.data_ptr(), begin, end, table.ptr, table.nseg,
                              _native.ms_dtype(mdtype), stream())
    _native.check(rc, "ms_cast_to_model")
    torch.cuda.synchronize()


__all__ = [name for name in dir() if not name.startswith("_")] + ["adamw_params"]


def master_step_within_ulps(before, got, want, m, v, *, lr, betas, eps, wd, step, ulps=2.0):
    """Per-step master check of the GPU (``got``) against the oracle
    (``want``), both started from ``before``, with ``m`` / ``v`` the step's
    new moments (equal on both sides, bit for bit; the callers assert that)
    and the step's hyper-parameters.

    The last part of the update, p + (-lr * (m / bc1)) / (sqrt(v / bc2) +
    eps) after the decay, is recomputed from the moments twice: with CPU
    torch's sqrt, which must give the oracle's masters bit for bit, and with
    a correctly rounded sqrt, which must give the GPU's bit for bit.  Then
    |got - want| <= ulps * spacing(want) per element, except where torch's
    sqrt is not correctly rounded (about 0.6% of its inputs): there the two
    updates differ by construction, and the GPU is the exactly rounded one.
    Returns (ok, worst ratio to spacing(want) over the elements whose sqrt
    agrees, number of elements over the bound whose sqrt differs)."""
    from oracle import recipe

    f = np.float32
    b1, b2 = float(betas[0]), float(betas[1])
    before = np.asarray(before, dtype=f)
    got = np.asarray(got, dtype=f)
    want = np.asarray(want, dtype=f)
    m = np.asarray(m, dtype=f)
    v = np.asarray(v, dtype=f)
    p1 = recipe.fma32(before, f(-lr * wd), before) if wd != 0.0 else before
    q = v / f(1.0 - b2 ** step)
    den_cpu = torch.from_numpy(q.copy()).sqrt().numpy() + f(eps)   # the oracle's sqrt
    den_rn = np.sqrt(q) + f(eps)
    num = f(-lr) * (m / f(1.0 - b1 ** step))
    if not np.array_equal((p1 + num / den_cpu).view(np.int32), want.view(np.int32)):
        return False, float("inf"), -1          # the oracle is not this update
    if not np.array_equal((p1 + num / den_rn).view(np.int32), got.view(np.int32)):
        return False, float("inf"), -2          # the GPU is not the exactly rounded update
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    ratio = diff / np.spacing(np.abs(want)).astype(np.float64)
    sqrt_differs = den_cpu != den_rn
    over = ratio > ulps
    if np.any(over & ~sqrt_differs):
        return False, float(ratio[~sqrt_differs].max()), int(np.sum(over & sqrt_differs))
    worst = float(ratio[~sqrt_differs].max()) if np.any(~sqrt_differs) else 0.0
    return True, worst, int(np.sum(over))


def step_hyper(engine, gi: int = 0) -> dict:
    """Group ``gi``'s AdamW hyper-parameters for the step about to run (read
    before ``engine.step()``: the scheduler moves lr afterwards) and the
    step count that step will use."""
    from minispeed_amd.optim.adam import FlatAdam

    lr, betas, eps, wd = FlatAdam.hyper(engine.optimizer.param_groups[gi])
    return dict(lr=lr, betas=betas, eps=eps, wd=wd, step=int(engine.optimizer.state[gi]["step"]) + 1)


def clip_override(engine):
    """The GPU boundary's clip decision and coefficient, for the oracle's
    ``step(clip_override=...)``: the oracle then runs its AdamW arithmetic on
    exactly the gradients the GPU clipped, so moments must match bit for bit
    and masters within 2 fp32 ulp per step (the norm is checked on its own,
    to 1e-5)."""
    lb = engine.last_boundary
    return bool(lb.clip_applied), float(lb.coef64)


def relative_within(got, want, scale, rtol=1e-5):
    """Per element |got - want| <= rtol * max(|want|, scale), with ``scale``
    the element's largest magnitude along its trajectory: relative to the
    element's own size, also where it passes near zero on the way.  Returns
    (ok, worst ratio of the difference to its bound)."""
    got = np.asarray(got, dtype=np.float32).astype(np.float64)
    want64 = np.asarray(want, dtype=np.float32).astype(np.float64)
    size = np.maximum(np.abs(want64), np.abs(np.asarray(scale, dtype=np.float32)).astype(np.float64))
    diff = np.abs(got - want64)
    bound = rtol * size
    ratio = np.where(diff == 0.0, 0.0, diff / np.maximum(bound, np.finfo(np.float64).tiny))
    worst = float(ratio.max()) if ratio.size else 0.0
    return worst <= 1.0, worst
