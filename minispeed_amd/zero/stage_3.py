"""ZeRO stage 3 on one GPU (minispeed/zero/stage_3.py).

Between steps every parameter is a flat model-dtype placeholder of its owned
slice and the masters are the owned shard; ``gather_parameters`` gives the
parameters their real shapes holding the cast of the masters (the
cast-on-gather, stage_3.py:67-86), ``free_parameters`` drops them back to
placeholders refreshed from the masters (stage_3.py:88-100).

The placeholders are views into one model-dtype buffer of the shard
(``FlatParamGroup.model_shard``), and at world size 1 the gathered
parameters are shaped views into the same buffer, so neither gather nor
free allocates.  The gather casts the masters into that buffer (K4) every
time, as the reference's gather does, so whatever was written into a freed
placeholder is overwritten.  With ``gather_reuse`` (the
``hip_boundary.stage3_gather_reuse`` option) the cast is skipped when the
buffer already holds the cast of the current masters by the version
counters of the masters and the parameters (``model_is_fresh``); writes
through a freed placeholder's ``.data`` are not seen by those counters and
then survive the gather.  In the fused boundary K3 writes the cast of the
updated masters straight into the buffer, which is what the reference's
Adam step followed by ``free_parameters`` leaves behind.  On a skipped step
the masters are unchanged and the buffer is refreshed by the cast kernel
instead.
"""

from __future__ import annotations

from typing import List, Optional

import torch

from .. import comm
from ..flat import FlatParamGroup
from .stage_1_and_2 import ZeROOptimizer


class ZeROStage3Optimizer(ZeROOptimizer):
    def __init__(self, flat_groups: List[FlatParamGroup], option_groups: List[dict]):
        super().__init__(flat_groups, option_groups, zero_stage=3)
        self._gathered = False
        # placeholders created for the current boundary (K3 writes them)
        self._boundary_freed = False
        # skip the gather's cast when the buffer is fresh (opt-in)
        self.gather_reuse = False

    @property
    def params_gathered(self) -> bool:
        return self._gathered

    @torch.no_grad()
    def gather_parameters(self) -> None:
        if self._gathered:
            return
        for g in self.flat_groups:
            if g.numel_shard() != g.numel_padded:
                raise comm.MultiGPUNotSupported(
                    "gathering a ZeRO-3 shard needs the other ranks' shards "
                    f"(shard {g.numel_shard()} of {g.numel_padded})"
                )
            g.materialize_params()
            if not (self.gather_reuse and g.model_is_fresh()):
                g.copy_flat_to_model()
        self._gathered = True

    @torch.no_grad()
    def free_parameters(self) -> None:
        if not self._gathered:
            return
        for g in self.flat_groups:
            g.dematerialize_params()
            g.copy_flat_to_model()
        self._gathered = False

    @torch.no_grad()
    def sync_parameters(self) -> None:
        self.free_parameters()

    @torch.no_grad()
    def step(self) -> bool:
        self.adam.step()     # marks the groups' model copies stale
        return True

    # ------------------------------------------------------ fused boundary
    @torch.no_grad()
    def reduce_gradients(self) -> None:
        """stage_3.py:120-126: the one-rank reduce-scatter into
        ``grad_shard``, then the full flat gradient is dropped."""
        super().reduce_gradients()
        for g in self.flat_groups:
            g.grad = None

    def _model_targets(self) -> List[Optional[List[int]]]:
        if not self._gathered:
            # the reference's free_parameters is a no-op then: nothing written
            self._boundary_freed = False
            return [None for _ in self.flat_groups]
        for g in self.flat_groups:
            g.dematerialize_params()
        self._boundary_freed = True
        return [g.model_pointers() for g in self.flat_groups]

    def _after_boundary(self, overflow: bool) -> None:
        if self._boundary_freed:
            for g in self.flat_groups:
                if overflow:
                    g.copy_flat_to_model()
                else:
                    g.model_written()     # K3 wrote the cast of the new masters
            self._gathered = False
            self._boundary_freed = False
        elif not overflow:
            for g in self.flat_groups:
                g.masters_written()       # placeholders keep the old values
        for g in self.flat_groups:
            if g._grad is not None:
                g.grad = None  # the full flat grad never outlives the boundary
