"""The fused boundary step: K1 (+ its tile fold) -> K2 -> K3 on the current
HIP stream with one device->host read-back.

Replaces the unfused sequence of minispeed's
``DeepSpeedEngine._take_optimizer_step`` (engine.py:268-322):

    flatten_grads            flat.py:196-213       \\
    has_overflow             precision.py:79-87     > K1 per group
    unscale_grads            flat.py:243-247       /   (+ sumsq per 2048-element tile, folded)
    reduce_gradients         stage_1_and_2.py:86-102   identity at world 1
    clip_gradients           stage_1_and_2.py:105-128  K2 (norm, coef, skip)
    FlatAdam.step            optim/adam.py:59-93   \\
    sync_parameters          stage_1_and_2.py:79-83 > K3 per group
    (stage 3) free_parameters  stage_3.py:88-110   /
    DynamicLossScaler.update precision.py:50-62        K2 (checked on host)

K3 is gated on the device overflow flag, so the launch sequence does not
wait for the host: the only synchronisation is the final copy of the
``ms_step_scalars_t`` K2 wrote.
"""

from __future__ import annotations

import ctypes
import time
from dataclasses import dataclass
from typing import Callable, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _native
from .flat import FlatParamGroup, record_streams


def _f32(x: float) -> float:
    """x rounded to fp32 (round to nearest even), as a Python float."""
    return ctypes.c_float(x).value


def adamw_params(
    lr: float, betas: Sequence[float], eps: float, weight_decay: float, step: int,
    grad_scale: float = 1.0, unscale: bool = False,
) -> _native.AdamWParams:
    """Round this step's AdamW scalars the way the torch op sequence of
    optim/adam.py:72-91 does: every Python double becomes fp32 at the op that
    consumes it.  The doubles are computed here and stored into the
    ``c_float`` fields of the struct, a C double -> float conversion that
    rounds to nearest even, as ``np.float32`` does."""
    lr = float(lr)
    beta1, beta2 = (float(b) for b in betas)
    wd = float(weight_decay)
    return _native.AdamWParams(
        neg_lr=-lr,
        decay_alpha=-lr * wd,
        beta1=beta1,
        one_minus_beta1=1.0 - beta1,
        beta2=beta2,
        one_minus_beta2=1.0 - beta2,
        bias_c1=1.0 - beta1 ** step,
        bias_c2=1.0 - beta2 ** step,
        eps=float(eps),
        grad_scale=float(grad_scale),
        decay=1 if wd != 0.0 else 0,
        unscale=_native.SCALE_DIVIDE if unscale else _native.SCALE_NONE,
    )


class HostReadback:
    """K2's result in pinned host memory, read without a copy and without
    anything between K2 and K3 in the stream.

    ``arm()`` clears the struct's ``ready`` word before K2 is launched with
    ``ptr`` as its host output; K2 writes the struct, makes it visible
    system-wide and then sets ``ready``; ``wait()`` polls that word (K3, queued
    behind K2, keeps running) and returns the struct.  An event recorded
    after K2 for the host to wait on put a 4-5.5 us gap between K2 and K3.
    If the word does not turn within ``patience`` seconds (a deep queue of
    earlier work), the stream is synchronised instead, which also reports a
    device error."""

    _READY = _native.StepScalars.ready.offset

    def __init__(self, patience: float = 5.0):
        self.host = torch.empty(_native.SCALARS_BYTES, dtype=torch.uint8, pin_memory=True)
        self._bytes = self.host.numpy()
        self._ready = self._bytes[self._READY:self._READY + 4].view(np.uint32)
        self.patience = patience

    @property
    def ptr(self) -> int:
        return self.host.data_ptr()

    def arm(self) -> None:
        self._ready[0] = 0

    def wait(self, stream: int) -> _native.StepScalars:
        ready = self._ready
        spins = 0
        deadline = None
        while ready[0] != 1:
            spins += 1
            if spins & 0x3FF == 0:
                now = time.perf_counter()
                if deadline is None:
                    deadline = now + self.patience
                elif now > deadline:
                    _native.hip_check(_native.hip_runtime().hipStreamSynchronize(stream),
                                      "hipStreamSynchronize")
                    if ready[0] != 1:
                        raise RuntimeError("the norm/clip kernel's host result did not arrive")
                    break
        return _native.StepScalars.from_buffer_copy(self._bytes.tobytes())


class Workspace:
    """Device scratch of the boundary step (no allocation per step)."""

    def __init__(self, device: torch.device, ngroups: int):
        self.device = device
        self.nblk = _native.stats_blocks()
        self.ngroups = ngroups
        n = max(1, ngroups) * self.nblk
        self.partials = torch.empty(n, dtype=torch.float64, device=device)
        self.flags = torch.empty(n, dtype=torch.int32, device=device)
        self.scalars = torch.empty(_native.SCALARS_BYTES, dtype=torch.uint8, device=device)
        # K1's tile slots, shared by the groups of a boundary (each group's
        # K1 and fold run before the next group's K1, on one stream); grown
        # on demand, with every stream that used them recorded
        self.tile_sums: Optional[torch.Tensor] = None
        self.tile_flags: Optional[torch.Tensor] = None
        self._tile_streams: set = set()
        # K2 also writes its result to pinned host memory, which the host
        # polls (HostReadback): no copy, and K3, queued behind K2, keeps
        # running while the host does its bookkeeping
        self.readback = HostReadback()
        self.host = self.readback.host
        self._stream: Optional[torch.cuda.Stream] = None   # stream of the last boundary

    def partial_ptrs(self, g: int):
        off = g * self.nblk
        return (
            self.partials.data_ptr() + off * 8,
            self.flags.data_ptr() + off * 4,
        )

    def tile_ptrs(self, ntiles: int):
        """Addresses (sums, flags) of at least ``ntiles`` K1 tile slots for
        kernels on the current stream."""
        if self.tile_sums is None or self.tile_sums.numel() < ntiles:
            # the replaced buffers' memory stays with the streams recorded on
            # them until those have run what was queued there
            self.tile_sums = torch.empty(max(1, ntiles), dtype=torch.float64, device=self.device)
            self.tile_flags = torch.empty(max(1, ntiles), dtype=torch.int32, device=self.device)
            self._tile_streams = set()
        cur = torch.cuda.current_stream(self.device)
        if cur.cuda_stream not in self._tile_streams:
            self.tile_sums.record_stream(cur)
            self.tile_flags.record_stream(cur)
            self._tile_streams.add(cur.cuda_stream)
        return self.tile_sums.data_ptr(), self.tile_flags.data_ptr()

    def read_scalars(self) -> _native.StepScalars:
        """Copy K2's result to pinned memory and wait for the stream."""
        self.host.copy_(self.scalars, non_blocking=True)
        torch.cuda.current_stream(self.device).synchronize()
        return _native.StepScalars.from_buffer_copy(self.host.numpy().tobytes())

    def enter(self) -> torch.cuda.Stream:
        """Called at the start of a boundary; returns the current stream,
        which the boundary's kernels run on.  Kernels of the previous
        boundary (K3 reading the scalars and segment tables this boundary
        overwrites) may still run on its stream; if the current stream is
        another one, it first waits for everything queued there."""
        cur = torch.cuda.current_stream(self.device)
        if self._stream is not None and self._stream != cur:
            cur.wait_stream(self._stream)
        self._stream = cur
        return cur

    def finish_readback(self) -> _native.StepScalars:
        """Wait for K2's scalars in pinned host memory (later kernels on the
        stream keep running)."""
        return self.readback.wait(self._stream.cuda_stream)


class LaunchTimer:
    """Optional HIP-event timing of the boundary kernels.

    When attached to an optimizer (``optimizer.launch_timer``), every K1 /
    K2 / K3 launch is bracketed by events recorded on the current stream,
    the stream the kernels run on.  The events are created with
    ``hipEventDisableSystemFence``: a default event performs a system-scope
    release when it is recorded (a cache write-back between the kernels it
    brackets, 10-15 us per event between the boundary kernels), which the
    timing-only events do without, so the timed kernels run back to back as
    in an untimed step.  ``durations_ms(name)`` is valid after the device
    has been synchronised.  ``reserve(n)`` creates n events up front, so
    that a timed region pays only for recording them.
    """

    def __init__(self, reserve: int = 0):
        self._hip = _native.hip_runtime()
        self._events = {}
        self._pool: List[int] = []
        self._owned: List[int] = []
        self.reserve(reserve)

    def _create(self) -> int:
        ev = ctypes.c_void_p()
        _native.hip_check(self._hip.hipEventCreateWithFlags(
            ctypes.byref(ev), _native.HIP_EVENT_DISABLE_SYSTEM_FENCE), "hipEventCreateWithFlags")
        self._owned.append(ev.value)
        return ev.value

    def reserve(self, n: int) -> None:
        self._pool.extend(self._create() for _ in range(n))

    def _record(self) -> int:
        ev = self._pool.pop() if self._pool else self._create()
        stream = torch.cuda.current_stream().cuda_stream
        _native.hip_check(self._hip.hipEventRecord(ev, stream), "hipEventRecord")
        return ev

    def start(self, name: str):
        return (name, self._record())

    def stop(self, token) -> None:
        name, start = token
        self._events.setdefault(name, []).append((start, self._record()))

    def durations_ms(self, name: str) -> List[float]:
        out = []
        for a, b in self._events.get(name, []):
            ms = ctypes.c_float()
            _native.hip_check(self._hip.hipEventElapsedTime(ctypes.byref(ms), a, b),
                              "hipEventElapsedTime")
            out.append(float(ms.value))
        return out

    def reset(self) -> None:
        """Forget the recorded pairs (their events go back to the pool)."""
        for pairs in self._events.values():
            for a, b in pairs:
                self._pool.extend((a, b))
        self._events.clear()

    def __del__(self):
        hip = getattr(self, "_hip", None)
        for ev in getattr(self, "_owned", ()):
            hip.hipEventDestroy(ev)


class _NoTimer:
    def start(self, name):
        return None

    def stop(self, token):
        return None


_NO_TIMER = _NoTimer()


@dataclass
class GroupLaunch:
    """What K1/K3 need for one group at one boundary."""

    group: FlatParamGroup
    lr: float
    betas: Sequence[float]
    eps: float
    weight_decay: float
    step: int                     # Adam step number this update would use
    exp_avg: torch.Tensor         # owned-range moments (optim/adam.py:58-65)
    exp_avg_sq: torch.Tensor
    grads: Sequence[int]          # gradient address per parameter (0: none)
    grad_dtype: Optional[int] = None   # MS_DTYPE_* of the gradients (default: the params')
    # (sum-of-squares slots, flag slots, count) K5 left for the gradients
    # (contiguous mode): folded into the partial sums instead of the K1 scan
    tile_stats: Optional[Tuple[int, int, int]] = None


def run_boundary(
    launches: List[GroupLaunch],
    ws: Workspace,
    *,
    scaler,
    max_norm: Optional[float],
    materialize_flat_grad: bool,
    model_targets: Callable[[], List[Optional[List[int]]]],
    timer: Optional[LaunchTimer] = None,
    keep: Sequence[Optional[torch.Tensor]] = (),
) -> _native.StepScalars:
    """Launch the whole boundary and return K2's scalars (one host sync).

    K1 and K2 are launched as soon as the gradient addresses are known (K2
    writes its scalars to device memory for K3 and to pinned host memory
    for the host) and an event marks K2's end; ``model_targets()``
    (the addresses K3 casts the updated masters into, per group; ``None`` for
    no write) is called after that, so whatever it does on the host overlaps
    K1 on the device.  The function returns once K2's scalars are on the
    host, which is before K3 has finished: K3 runs on the current stream, so
    everything queued there afterwards is ordered after it.  ``keep`` holds
    the tensors behind ``GroupLaunch.grads``; the current stream is recorded
    on each, so the caller may drop them once this returns, whichever
    stream allocated them.
    """
    lib = _native.load()
    device = ws.device
    cur = ws.enter()
    stream = cur.cuda_stream
    scale = float(scaler.loss_scale_factor)
    unscale = scale != 1.0
    scale32 = _f32(scale)
    timer = timer or _NO_TIMER

    dtypes, flats = [], []
    for gi, gl in enumerate(launches):
        g = gl.group
        dtype = _native.ms_dtype(g.params[0].dtype)
        gdtype = dtype if gl.grad_dtype is None else gl.grad_dtype
        flat_out = None
        if materialize_flat_grad:
            flat_out = g.flat_grad_for_overwrite()      # K1 writes every element
        lo, hi = g.own_range
        gbytes = 4 if gdtype == _native.DTYPE_F32 else 2
        psum, pflag = ws.partial_ptrs(gi)
        if gl.tile_stats is not None and flat_out is None and (lo, hi) == (0, g.numel_padded):
            # the accumulation pass already scanned the sums: fold its tile
            # statistics into the partial slots (no second read of the sums)
            ts, tf, ntiles = gl.tile_stats
            tok = timer.start("k1")
            rc = lib.ms_reduce_tile_stats(ts or None, tf or None, ntiles, psum, pflag, ws.nblk, stream)
            timer.stop(tok)
            _native.check(rc, "ms_reduce_tile_stats")
        else:
            t1 = g.table("k1").upload(g.boundary_table(0, g.numel_padded, gl.grads, None, gbytes), cur)
            ntiles = _native.scan_tiles(g.numel_padded)
            tsum, tflag = ws.tile_ptrs(ntiles)
            tok = timer.start("k1")
            rc = lib.ms_grad_stats(
                t1[0], t1[1], gdtype, 0, g.numel_padded, lo, hi,
                _native.SCALE_DIVIDE if unscale else _native.SCALE_NONE, scale32,
                flat_out.data_ptr() if flat_out is not None else None,
                tsum, tflag, ntiles, psum, pflag, ws.nblk, stream,
            )
            timer.stop(tok)
            _native.check(rc, "ms_grad_stats")
        dtypes.append((gdtype, dtype, gbytes))
        flats.append(flat_out)

    ws.readback.arm()
    tok = timer.start("k2")
    rc = lib.ms_norm_clip(
        ws.partials.data_ptr(), ws.flags.data_ptr(), ws.nblk, len(launches),
        1 if max_norm is not None else 0, float(max_norm or 0.0),
        1 if scaler.enabled else 0, float(scaler.scale), int(scaler.good_steps),
        int(scaler.skipped_steps), int(scaler.scale_window),
        float(scaler.min_scale), float(scaler.max_scale),
        ws.scalars.data_ptr(), ws.readback.ptr, stream,
    )
    timer.stop(tok)
    _native.check(rc, "ms_norm_clip")

    models = model_targets()
    for gl, (gdtype, dtype, gbytes), flat_out, mptrs in zip(launches, dtypes, flats, models):
        g = gl.group
        lo, hi = g.own_range
        if hi <= lo:
            continue
        master = g.shard
        if master.numel() != hi - lo or gl.exp_avg.numel() != hi - lo or gl.exp_avg_sq.numel() != hi - lo:
            raise RuntimeError(
                f"grad/shard shape mismatch: owned range {hi - lo} vs master {master.numel()}, "
                f"moments {gl.exp_avg.numel()}/{gl.exp_avg_sq.numel()}"
            )
        t3 = g.table("k3").upload(g.boundary_table(lo, hi, gl.grads, mptrs, gbytes), cur)
        hp = adamw_params(gl.lr, gl.betas, gl.eps, gl.weight_decay, gl.step,
                          grad_scale=scale, unscale=unscale and flat_out is None)
        fg_ptr = flat_out.data_ptr() + lo * 4 if flat_out is not None else None
        tok = timer.start("k3")
        rc = lib.ms_fused_adamw(
            master.data_ptr(), gl.exp_avg.data_ptr(), gl.exp_avg_sq.data_ptr(), fg_ptr,
            t3[0], t3[1], gdtype, dtype, lo, hi, ctypes.byref(hp), ws.scalars.data_ptr(), stream,
        )
        timer.stop(tok)
        _native.check(rc, "ms_fused_adamw")

    # The gradients may come from another stream (the one backward ran on):
    # once the caller drops them, the caching allocator could hand their
    # memory to that stream while K1 / K3 still read it here.  Recording
    # this stream on them defers the reuse until everything queued here so
    # far has run.  Done while K1 / K2 run, before the host waits.
    record_streams(keep, cur)
    return ws.finish_readback()


# ------------------------------------------------------------------ utility
def _whole_buffer_table(flat: torch.Tensor) -> torch.Tensor:
    """Device segment table of one row covering a contiguous buffer."""
    table = np.array([[0, flat.numel(), flat.data_ptr(), 0]], dtype=np.int64)
    return torch.from_numpy(table).to(flat.device)


def scale_in_place(buf: torch.Tensor, mode: int, factor: float) -> None:
    """``buf.div_(factor)`` (mode SCALE_DIVIDE, flat.py:243-247) or
    ``buf.mul_(factor)`` (mode SCALE_MULTIPLY, flat.py:249-257) of a
    contiguous fp32 device buffer, in place by K1, with ``factor`` rounded to
    fp32 first as torch does with a Python scalar."""
    _native.require_hip_tensor(buf, "scaled buffer")
    if buf.dtype != torch.float32 or not buf.is_contiguous():
        raise TypeError("scale_in_place needs a contiguous float32 buffer")
    n = buf.numel()
    if n == 0:
        return
    table = _whole_buffer_table(buf)
    _native.check(_native.load().ms_grad_stats(
        table.data_ptr(), 1, _native.DTYPE_F32, 0, n, 0, 0, mode, float(np.float32(factor)),
        buf.data_ptr(), None, None, 0, None, None, 0, _native.stream_handle(buf.device)),
        "ms_grad_stats(scale)")


def sumsq_device(buf: torch.Tensor) -> torch.Tensor:
    """``buf.pow(2).sum()`` as a 0-dim fp32 device tensor (flat.py:232-234):
    K1's fp64 tile partials, folded into K2's slots, summed by K2 and rounded
    to fp32 once."""
    _native.require_hip_tensor(buf, "sum-of-squares buffer")
    flat = buf.detach().reshape(-1)
    if not flat.is_contiguous():
        flat = flat.contiguous()
    n = flat.numel()
    if n == 0:
        return torch.zeros((), dtype=torch.float32, device=flat.device)
    lib = _native.load()
    ws = Workspace(flat.device, 1)
    table = _whole_buffer_table(flat)
    stream = _native.stream_handle(flat.device)
    psum, pflag = ws.partial_ptrs(0)
    ntiles = _native.scan_tiles(n)
    tsum, tflag = ws.tile_ptrs(ntiles)
    _native.check(lib.ms_grad_stats(table.data_ptr(), 1, _native.ms_dtype(flat.dtype), 0, n, 0, n, 0,
                                    1.0, None, tsum, tflag, ntiles, psum, pflag, ws.nblk, stream),
                  "ms_grad_stats")
    _native.check(lib.ms_norm_clip(psum, pflag, ws.nblk, 1, 0, 0.0, 0, 1.0, 0, 0, 1, 1.0, 1.0,
                                   ws.scalars.data_ptr(), None, stream), "ms_norm_clip")
    off = _native.StepScalars.sumsq.offset
    return ws.scalars[off:off + 4].view(torch.float32).clone().reshape(())


def scan_nonfinite(buf: torch.Tensor) -> bool:
    """inf/nan test of one device buffer with K1 + K2 (used by
    precision.has_overflow)."""
    _native.require_hip_tensor(buf, "has_overflow buffer")
    flat = buf.detach().reshape(-1)
    if not flat.is_contiguous():
        flat = flat.contiguous()
    n = flat.numel()
    dtype = _native.ms_dtype(flat.dtype)
    lib = _native.load()
    ws = Workspace(flat.device, 1)
    dev_table = _whole_buffer_table(flat)
    stream = _native.stream_handle(flat.device)
    psum, pflag = ws.partial_ptrs(0)
    ntiles = _native.scan_tiles(n)
    tsum, tflag = ws.tile_ptrs(ntiles)
    _native.check(lib.ms_grad_stats(dev_table.data_ptr(), 1, dtype, 0, n, 0, 0, 0, 1.0,
                                    None, tsum, tflag, ntiles, psum, pflag, ws.nblk, stream),
                  "ms_grad_stats")
    _native.check(lib.ms_norm_clip(psum, pflag, ws.nblk, 1, 0, 0.0, 0, 1.0, 0, 0, 1, 1.0, 1.0,
                                   ws.scalars.data_ptr(), None, stream), "ms_norm_clip")
    return bool(ws.read_scalars().overflow)
