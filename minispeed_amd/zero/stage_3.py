"""ZeRO stage 3 on one GPU (minispeed/zero/stage_3.py).

Between steps every parameter is a flat model-dtype placeholder of its owned
slice and the masters are the owned shard; ``gather_parameters`` gives the
parameters their real shapes and casts the masters into them (the
cast-on-gather, stage_3.py:67-86), ``free_parameters`` drops them back to
placeholders refreshed from the masters (stage_3.py:88-100).

In the fused boundary the placeholders are created before K3 runs and K3
writes the cast of the updated masters straight into them, which is what
the reference's Adam step followed by ``free_parameters`` leaves behind.  On
a skipped step the masters are unchanged and the placeholders are filled by
the cast kernel instead.  At world size 1 the all-gather is the identity, so
the gather casts from the master shard directly instead of through a
transient full fp32 copy: the cast is elementwise, the result identical.
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
            g.copy_flat_to_model(g.data)
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
        self.adam.step()
        return True

    # ------------------------------------------------------ fused boundary
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
            if overflow:
                for g in self.flat_groups:
                    g.copy_flat_to_model()
            self._gathered = False
            self._boundary_freed = False
        for g in self.flat_groups:
            if g.grad is not None:
                g.grad = None  # the full flat grad never outlives the boundary
