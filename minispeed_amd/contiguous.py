"""Opt-in contiguous gradients: fp32 accumulation into one flat buffer.

minispeed accumulates the micro-batch gradients of a window in
``param.grad``, in the parameter dtype (autograd under engine.py:235-251),
and copies them into the fp32 flat buffer at the boundary (flat.py:196-213).
With ``"hip_boundary": {"contiguous_gradients": true}`` a post-accumulate-grad
hook on every parameter takes the gradient backward has just produced and
releases ``param.grad``; the queued gradients are added, in fp32, into the
parameters' slices of one flat buffer per group by K5 in batches
(``ms_accumulate_grads``, up to 64 gradients per launch): when a bucket of
queued elements fills, and at the end of every backward pass (an autograd
final callback).  K5 runs on the stream current when the batch is flushed:
the gradients of one backward are assumed to come from that stream, as
autograd's do when the forward ran on one stream.

The same K5 pass also does the boundary scan's work on the new sums: for
every 2048-element tile of a parameter's slice it writes the fp64 sum of
squares of the unscaled sums and an inf/nan flag into the tile's slot.
The last K5 that touched a tile always left the statistics of its current
sums, and the slots are zeroed when a window starts (parameters without a
gradient count as zeros), so at the boundary the slots are folded into the
norm's partial sums (``ms_reduce_tile_stats``) and the fp32 sums are not
read a second time: the boundary moves 30 B/param (K3) instead of 34.
When the loss scale that unscaled the statistics is not the boundary's
(it changed inside the window), the boundary scans the sums again.

K5's tiles are 2048-element pieces of each parameter's slice, K1's are
2048-element pieces of the flat space; where a parameter does not start on
a multiple of 2048 the two tilings group the elements differently, so the
fp64 partial sums are added in another order and the norm (with it the clip
coefficient, and the masters where clipping applies) can differ from a K1
scan of the same sums in the last bit of the fp32 norm.  Both orders are
fixed: each path is run-to-run deterministic, and the tests hold the two
within 1.2e-7 relative of each other and within 1e-5 of the oracle.

Differences from minispeed, which is why the mode is off by default:

* sums are rounded to fp32 after each micro-batch instead of to the
  parameter dtype, so with fp16 / bf16 models the gradients (and everything
  after them) differ in the last bits, and a window whose half-precision sum
  would overflow does not;
* ``param.grad`` is ``None`` between micro-batches;
* the hooks move 6 (first micro-batch) or 10 B/param per micro-batch, the
  boundary 30 B/param (K3 reads 4-byte sums instead of 2-byte gradients).

Parameters that received no gradient in a window count as zeros, as in
minispeed: their segment-table rows carry no gradient address.
"""

from __future__ import annotations

import ctypes
from typing import Callable, List, Optional, Tuple

import numpy as np
import torch

from . import _native
from .flat import FlatParamGroup, record_streams


# K5's row layout (ms_accum_row_t) as a numpy record
ACCUM_ROW = np.dtype([("dst", np.int64), ("src", np.int64), ("numel", np.int64),
                      ("first", np.int32), ("reserved", np.int32),
                      ("tile_sumsq", np.int64), ("tile_flag", np.int64)])
assert ACCUM_ROW.itemsize == ctypes.sizeof(_native.AccumRow)

# queued gradient elements that trigger a flush inside backward (512 MB of
# half gradients): bounds what the queue holds on to
BUCKET_ELEMENTS = 1 << 28


def accumulate_rows(rows: np.ndarray, src_dtype: int, device: torch.device,
                    unscale: int = _native.SCALE_NONE, scale: float = 1.0) -> None:
    """K5 over a batch of ACCUM_ROW records (host memory) on the current
    stream of ``device``; rows with statistics slots are unscaled by
    ``scale`` (``unscale``: SCALE_NONE or SCALE_DIVIDE) for them."""
    if len(rows) == 0:
        return
    rows = np.ascontiguousarray(rows, dtype=ACCUM_ROW)
    rc = _native.load().ms_accumulate_grads(rows.ctypes.data, len(rows), src_dtype, unscale,
                                            ctypes.c_float(scale).value,
                                            _native.stream_handle(device))
    _native.check(rc, "ms_accumulate_grads")


def unscale_of(scale: float) -> Tuple[int, float]:
    """(unscale mode, fp32 scale) with which the boundary unscales gradients
    for the loss scale ``scale``."""
    return ((_native.SCALE_DIVIDE if scale != 1.0 else _native.SCALE_NONE),
            ctypes.c_float(scale).value)


class ContiguousGradients:
    def __init__(self, groups: List[FlatParamGroup], bucket_elements: int = BUCKET_ELEMENTS,
                 scale_fn: Optional[Callable[[], float]] = None):
        self.groups = groups
        self.window = 0
        self.bucket_elements = int(bucket_elements)
        # the loss scale the boundary will unscale by (the engine's scaler)
        self.scale_fn = scale_fn or (lambda: 1.0)
        # fold the K5 tile statistics at the boundary (False: scan the sums)
        self.use_tile_stats = True
        self.accum = [torch.empty(g.numel_padded, dtype=torch.float32, device=g.device)
                      for g in groups]
        self._offsets = [np.asarray(g.layout.offsets, dtype=np.int64) for g in groups]
        # statistics slots: parameter k of group g owns ceil(numel / 2048)
        # tiles from _tile0[g][k]
        tile = _native.ACCUM_TILE
        self._tile0, self.tile_sumsq, self.tile_flag = [], [], []
        for g in groups:
            counts = (np.asarray(g._numels, dtype=np.int64) + tile - 1) // tile
            self._tile0.append(np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.int64))
            n = int(counts.sum())
            self.tile_sumsq.append(torch.zeros(n, dtype=torch.float64, device=g.device))
            self.tile_flag.append(torch.zeros(n, dtype=torch.int32, device=g.device))
        # the (unscale, fp32 scale) of this window's flushes; None before the
        # first, False once two differed
        self._window_unscale = None
        # the stream of the last boundary (the sums and slots were read and
        # cleared there): a flush on another stream waits for it first
        self._boundary_stream: Optional[torch.cuda.Stream] = None
        # window in which each parameter last contributed (-1: never)
        self._seen = [np.full(len(g.params), -1, dtype=np.int64) for g in groups]
        # queued (group, index, gradient, first) in hook order, not yet added
        self._queue: List[Tuple[int, int, torch.Tensor, bool]] = []
        self._queued = set()
        self._queued_numel = 0
        self._callback_pending = False
        self._handles = []
        for gi, g in enumerate(groups):
            for k, p in enumerate(g.params):
                self._handles.append(p.register_post_accumulate_grad_hook(self._hook(gi, k)))

    def _hook(self, gi: int, k: int):
        def hook(param: torch.nn.Parameter) -> None:
            self.accumulate(gi, k, param)
            if not self._callback_pending:
                # runs once the whole backward is done (after autograd has
                # synchronised its streams with the caller's)
                self._callback_pending = True
                torch.autograd.Variable._execution_engine.queue_callback(self._end_of_backward)
        return hook

    def _end_of_backward(self) -> None:
        self._callback_pending = False
        self.flush()

    @torch.no_grad()
    def accumulate(self, gi: int, k: int, param: torch.nn.Parameter) -> None:
        """Queue ``param.grad`` for its fp32 slice and release it (K5 adds it
        at the next :meth:`flush`)."""
        grad = param.grad
        if grad is None:
            return
        g = self.groups[gi]
        n = g._numels[k]
        if grad.numel() != n:
            raise RuntimeError(f"gradient of a parameter has {grad.numel()} elements, expected {n}")
        _native.require_hip_tensor(grad, "gradient")
        if grad.device != g.device:
            raise RuntimeError(f"gradient on {grad.device}, expected {g.device}")
        _native.ms_dtype(grad.dtype)        # f32 / f16 / bf16 only
        if (gi, k) in self._queued:
            self.flush()                    # its earlier gradient goes first
        self._queue.append((gi, k, grad.contiguous(), self._seen[gi][k] != self.window))
        self._queued.add((gi, k))
        self._queued_numel += n
        self._seen[gi][k] = self.window
        param.grad = None
        if self._queued_numel >= self.bucket_elements:
            self.flush()

    @torch.no_grad()
    def flush(self) -> None:
        """Add every queued gradient into its slice, with its tiles'
        statistics: one batched K5 call per (device, gradient dtype), then
        drop the gradients."""
        if not self._queue:
            return
        queue, self._queue = self._queue, []
        self._queued.clear()
        self._queued_numel = 0
        unscale = unscale_of(float(self.scale_fn()))
        if self._window_unscale is None:
            self._window_unscale = unscale
        elif self._window_unscale != unscale:
            self._window_unscale = False
        batches = {}
        for gi, k, grad, first in queue:
            batches.setdefault((self.groups[gi].device, grad.dtype), []).append((gi, k, grad, first))
        for (device, dtype), items in batches.items():
            cur = torch.cuda.current_stream(device)
            prev = self._boundary_stream
            if prev is not None and prev.device == device and prev != cur:
                cur.wait_stream(prev)
            rows = np.zeros(len(items), dtype=ACCUM_ROW)
            rows["dst"] = [self.accum[gi].data_ptr() + int(self._offsets[gi][k]) * 4
                           for gi, k, _, _ in items]
            rows["src"] = [grad.data_ptr() for _, _, grad, _ in items]
            rows["numel"] = [grad.numel() for _, _, grad, _ in items]
            rows["first"] = [1 if first else 0 for _, _, _, first in items]
            rows["tile_sumsq"] = [self.tile_sumsq[gi].data_ptr() + int(self._tile0[gi][k]) * 8
                                  for gi, k, _, _ in items]
            rows["tile_flag"] = [self.tile_flag[gi].data_ptr() + int(self._tile0[gi][k]) * 4
                                 for gi, k, _, _ in items]
            accumulate_rows(rows, _native.ms_dtype(dtype), device, unscale[0], unscale[1])
            # the gradients' memory goes back to the caching allocator, which
            # hands it out again only in the order of this stream
            record_streams([grad for _, _, grad, _ in items], cur)

    def grad_pointers(self, gi: int) -> np.ndarray:
        """Addresses of the fp32 sums of group ``gi`` (0 for parameters
        without a gradient this window), with the padding row's trailing 0."""
        self.flush()
        seen = self._seen[gi] == self.window
        ptrs = np.zeros(len(self.groups[gi].params) + 1, dtype=np.int64)
        ptrs[:-1] = np.where(seen, self.accum[gi].data_ptr() + self._offsets[gi] * 4, 0)
        return ptrs

    def tile_stats(self, gi: int, scale: float) -> Optional[Tuple[int, int, int]]:
        """(sum-of-squares slots, flag slots, slot count) of group ``gi``
        for a boundary that unscales by ``scale``, or None when they cannot
        stand in for a scan of the sums (switched off, or this window's
        flushes unscaled by another scale)."""
        self.flush()
        if not self.use_tile_stats:
            return None
        w = self._window_unscale
        if w is False or (w is not None and w != unscale_of(float(scale))):
            return None
        return (self.tile_sumsq[gi].data_ptr(), self.tile_flag[gi].data_ptr(),
                int(self.tile_sumsq[gi].numel()))

    def next_window(self) -> None:
        """Forget the sums (the boundary consumed them, or zero_grad): the
        statistics slots are cleared on the current stream; queued
        gradients of the abandoned window are dropped unread."""
        self._queue = []
        self._queued.clear()
        self._queued_numel = 0
        self._callback_pending = False
        self._window_unscale = None
        for ts, tf in zip(self.tile_sumsq, self.tile_flag):
            ts.zero_()
            tf.zero_()
        if self.groups:
            self._boundary_stream = torch.cuda.current_stream(self.groups[0].device)
        self.window += 1

    def remove(self) -> None:
        for h in self._handles:
            h.remove()
        self._handles = []
