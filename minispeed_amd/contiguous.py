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
final callback).  The boundary then reads the fp32 sums through the same
segment tables (K1 and K3 with fp32 gradients).  K5 runs on the stream
current when the batch is flushed: the gradients of one backward are
assumed to come from that stream, as autograd's do when the forward ran on
one stream.

Differences from minispeed, which is why the mode is off by default:

* sums are rounded to fp32 after each micro-batch instead of to the
  parameter dtype, so with fp16 / bf16 models the gradients (and everything
  after them) differ in the last bits, and a window whose half-precision sum
  would overflow does not;
* ``param.grad`` is ``None`` between micro-batches;
* the boundary reads 4 bytes per gradient element instead of 2 (34 B/param
  with half gradients against 30 in the default mode), plus 6 (first
  micro-batch) or 10 B/param per micro-batch in the hooks.

Parameters that received no gradient in a window count as zeros, as in
minispeed: their segment-table rows carry no gradient address.
"""

from __future__ import annotations

import ctypes
from typing import List, Tuple

import numpy as np
import torch

from . import _native
from .flat import FlatParamGroup, record_streams


# K5's row layout (ms_accum_row_t) as a numpy record
ACCUM_ROW = np.dtype([("dst", np.int64), ("src", np.int64), ("numel", np.int64),
                      ("first", np.int32), ("reserved", np.int32)])
assert ACCUM_ROW.itemsize == ctypes.sizeof(_native.AccumRow)

# queued gradient elements that trigger a flush inside backward (512 MB of
# half gradients): bounds what the queue holds on to
BUCKET_ELEMENTS = 1 << 28


def accumulate_rows(rows: np.ndarray, src_dtype: int, device: torch.device) -> None:
    """K5 over a batch of ACCUM_ROW records (host memory) on the current
    stream of ``device``."""
    if len(rows) == 0:
        return
    rows = np.ascontiguousarray(rows, dtype=ACCUM_ROW)
    rc = _native.load().ms_accumulate_grads(rows.ctypes.data, len(rows), src_dtype,
                                            _native.stream_handle(device))
    _native.check(rc, "ms_accumulate_grads")


class ContiguousGradients:
    def __init__(self, groups: List[FlatParamGroup], bucket_elements: int = BUCKET_ELEMENTS):
        self.groups = groups
        self.window = 0
        self.bucket_elements = int(bucket_elements)
        self.accum = [torch.empty(g.numel_padded, dtype=torch.float32, device=g.device)
                      for g in groups]
        self._offsets = [np.asarray(g.layout.offsets, dtype=np.int64) for g in groups]
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
        """Add every queued gradient into its slice: one batched K5 call per
        (device, gradient dtype), then drop the gradients."""
        if not self._queue:
            return
        queue, self._queue = self._queue, []
        self._queued.clear()
        self._queued_numel = 0
        batches = {}
        for gi, k, grad, first in queue:
            batches.setdefault((self.groups[gi].device, grad.dtype), []).append((gi, k, grad, first))
        for (device, dtype), items in batches.items():
            rows = np.zeros(len(items), dtype=ACCUM_ROW)
            rows["dst"] = [self.accum[gi].data_ptr() + int(self._offsets[gi][k]) * 4 for gi, k, _, _ in items]
            rows["src"] = [grad.data_ptr() for _, _, grad, _ in items]
            rows["numel"] = [grad.numel() for _, _, grad, _ in items]
            rows["first"] = [1 if first else 0 for _, _, _, first in items]
            accumulate_rows(rows, _native.ms_dtype(dtype), device)
            # the gradients' memory goes back to the caching allocator, which
            # hands it out again only in the order of this stream
            record_streams([grad for _, _, grad, _ in items], torch.cuda.current_stream(device))

    def grad_pointers(self, gi: int) -> np.ndarray:
        """Addresses of the fp32 sums of group ``gi`` (0 for parameters
        without a gradient this window), with the padding row's trailing 0."""
        self.flush()
        seen = self._seen[gi] == self.window
        ptrs = np.zeros(len(self.groups[gi].params) + 1, dtype=np.int64)
        ptrs[:-1] = np.where(seen, self.accum[gi].data_ptr() + self._offsets[gi] * 4, 0)
        return ptrs

    def next_window(self) -> None:
        """Forget the sums (the boundary consumed them, or zero_grad); queued
        gradients of the abandoned window are dropped unread."""
        self._queue = []
        self._queued.clear()
        self._queued_numel = 0
        self._callback_pending = False
        self.window += 1

    def remove(self) -> None:
        for h in self._handles:
            h.remove()
        self._handles = []
