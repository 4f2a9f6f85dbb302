"""Opt-in contiguous gradients: fp32 accumulation into one flat buffer.

minispeed accumulates the micro-batch gradients of a window in
``param.grad``, in the parameter dtype (autograd under engine.py:235-251),
and copies them into the fp32 flat buffer at the boundary (flat.py:196-213).
With ``"hip_boundary": {"contiguous_gradients": true}`` a post-accumulate-grad
hook on every parameter adds the gradient backward has just produced, in
fp32, into the parameter's slice of one flat buffer per group (K5,
``ms_accumulate_grad``) and releases ``param.grad``.  The boundary then
reads the fp32 sums through the same segment tables (K1 and K3 with fp32
gradients).

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

from typing import List

import numpy as np
import torch

from . import _native
from .flat import FlatParamGroup


class ContiguousGradients:
    def __init__(self, groups: List[FlatParamGroup]):
        self.groups = groups
        self.window = 0
        self.accum = [torch.empty(g.numel_padded, dtype=torch.float32, device=g.device)
                      for g in groups]
        self._offsets = [np.asarray(g.layout.offsets, dtype=np.int64) for g in groups]
        # window in which each parameter last contributed (-1: never)
        self._seen = [np.full(len(g.params), -1, dtype=np.int64) for g in groups]
        self._handles = []
        for gi, g in enumerate(groups):
            for k, p in enumerate(g.params):
                self._handles.append(p.register_post_accumulate_grad_hook(self._hook(gi, k)))

    def _hook(self, gi: int, k: int):
        def hook(param: torch.nn.Parameter) -> None:
            self.accumulate(gi, k, param)
        return hook

    @torch.no_grad()
    def accumulate(self, gi: int, k: int, param: torch.nn.Parameter) -> None:
        """Add ``param.grad`` into its fp32 slice and release it."""
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
        grad = grad.contiguous()
        first = self._seen[gi][k] != self.window
        dst = self.accum[gi].data_ptr() + int(self._offsets[gi][k]) * 4
        rc = _native.load().ms_accumulate_grad(
            dst, grad.data_ptr(), _native.ms_dtype(grad.dtype), n, 1 if first else 0,
            _native.stream_handle(g.device))
        _native.check(rc, "ms_accumulate_grad")
        self._seen[gi][k] = self.window
        # the caching allocator reuses the released memory in stream order,
        # after the kernel just queued
        param.grad = None

    def grad_pointers(self, gi: int) -> np.ndarray:
        """Addresses of the fp32 sums of group ``gi`` (0 for parameters
        without a gradient this window), with the padding row's trailing 0."""
        seen = self._seen[gi] == self.window
        ptrs = np.zeros(len(self.groups[gi].params) + 1, dtype=np.int64)
        ptrs[:-1] = np.where(seen, self.accum[gi].data_ptr() + self._offsets[gi] * 4, 0)
        return ptrs

    def next_window(self) -> None:
        """Forget the sums (the boundary consumed them, or zero_grad)."""
        self.window += 1

    def remove(self) -> None:
        for h in self._handles:
            h.remove()
        self._handles = []
