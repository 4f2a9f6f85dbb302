"""ZeRO stages 0/1/2 on one GPU (minispeed/zero/stage_1_and_2.py).

At world size 1 the stages differ only in which flat buffers exist: stage 0
and 1 are identical (the all-gather after the step is skipped, reference
stage_1_and_2.py:139-145), stage 2 adds the ``grad_shard`` buffer that the
world-1 reduce-scatter would copy into (stage_1_and_2.py:95-96).  The
boundary step is the fused K1 -> K2 -> K3 sequence of ``boundary.py``; the
fused path never materialises the flat gradient, so ``grad`` and
``grad_shard`` stay the zeros the reference leaves in them after its
``zero_grad``.
"""

from __future__ import annotations

from typing import List, Optional

import torch

from .. import _native, comm
from ..boundary import GroupLaunch, LaunchTimer, Workspace, run_boundary
from ..flat import FlatParamGroup
from ..optim.adam import FlatAdam


class ZeROOptimizer:
    def __init__(self, flat_groups: List[FlatParamGroup], option_groups: List[dict], zero_stage: int = 0):
        if zero_stage not in (0, 1, 2, 3):
            raise ValueError(f"Unsupported ZeRO stage: {zero_stage}")
        self.flat_groups = flat_groups
        self.zero_stage = zero_stage
        self.world_size = comm.get_world_size()
        self.rank = comm.get_rank()
        self.adam = FlatAdam(flat_groups, option_groups, zero_stage=zero_stage)
        self.grad_norm: Optional[float] = None
        self._workspace: Optional[Workspace] = None
        self.launch_timer: Optional[LaunchTimer] = None  # HIP-event timing hook
        # opt-in fp32 gradient accumulation (contiguous.py); set by the engine
        self.contiguous = None

    # ------------------------------------------------------ torch-ish surface
    @property
    def param_groups(self) -> List[dict]:
        return self.adam.param_groups

    @property
    def state(self) -> List[dict]:
        return self.adam.state

    def zero_grad(self) -> None:
        for g in self.flat_groups:
            g.zero_grad()

    # --------------------------------------------- parameter materialization
    @property
    def params_gathered(self) -> bool:
        return True

    @torch.no_grad()
    def gather_parameters(self) -> None:
        """Stages 0-2 keep full parameters resident."""

    @torch.no_grad()
    def free_parameters(self) -> None:
        """Stages 0-2 keep full parameters resident."""

    @torch.no_grad()
    def sync_parameters(self) -> None:
        """Cast the masters into the model parameters (stage_1_and_2.py:79-83)."""
        for g in self.flat_groups:
            g.copy_flat_to_model()

    # ----------------------------------------- unfused step pieces (W = 1)
    @torch.no_grad()
    def reduce_gradients(self) -> None:
        """stage_1_and_2.py:86-102 at world size 1: stages 0/1 leave the
        flat gradient as it is (an all-reduce over one rank, no division),
        stage 2 copies it into ``grad_shard`` (the one-rank reduce-scatter)."""
        for g in self.flat_groups:
            if self.zero_stage >= 2:
                comm.reduce_scatter(g.grad_shard, g.grad)
                g._shard_dirty = True
            else:
                comm.all_reduce(g.grad)

    @torch.no_grad()
    def clip_gradients(self, max_norm: Optional[float]) -> float:
        """stage_1_and_2.py:105-128: the global L2 norm of the owned
        gradients (group sums of squares added in fp32, fp32 sqrt), and, if
        ``max_norm`` is set and the norm exceeds it, every group's owned
        gradients multiplied by ``max_norm / (norm + 1e-6)``."""
        total = torch.zeros((), dtype=torch.float32, device=self.flat_groups[0].device)
        for g in self.flat_groups:
            total += g.local_grad_sumsq()
        norm = float(total.sqrt().item())
        self.grad_norm = norm
        if max_norm is not None and norm > max_norm:
            coef = max_norm / (norm + 1e-6)
            for g in self.flat_groups:
                g.scale_grads(coef)
        return norm

    @torch.no_grad()
    def step(self) -> bool:
        """Unfused AdamW over already reduced/clipped grads (the reference's
        ``ZeROOptimizer.step``); the engine uses :meth:`boundary_step`."""
        return self.adam.step()

    # ------------------------------------------------------ fused boundary
    def _ws(self) -> Workspace:
        if self._workspace is None:
            self._workspace = Workspace(self.flat_groups[0].device, len(self.flat_groups))
        return self._workspace

    def _model_targets(self) -> List[Optional[List[int]]]:
        """Where K3 writes the model-dtype copy of each group (addresses of
        the parameters' storage)."""
        return [g.model_pointers() for g in self.flat_groups]

    def _after_boundary(self, overflow: bool) -> None:
        """Stage-specific follow-up once the scalars are on the host."""

    @torch.no_grad()
    def boundary_step(self, scaler, max_norm: Optional[float], materialize_flat_grad: bool = False):
        """Run flatten/flag/unscale/norm/clip/AdamW/cast for every group as
        K1 -> K2 -> K3 and return the host copy of K2's scalars.

        ``param.grad`` is released for every parameter (flat.py:213).  The
        Adam step counters advance only for an applied step (the caller
        commits them via :meth:`commit_step`).
        """
        ws = self._ws()
        keep: List[torch.Tensor] = []
        launches = []
        for gi, (g, group, state) in enumerate(zip(self.flat_groups, self.adam.param_groups,
                                                   self.adam.state)):
            grad_dtype = None
            tile_stats = None
            if self.contiguous is not None:
                ptrs, grad_dtype = self.contiguous.grad_pointers(gi), _native.DTYPE_F32
                tile_stats = self.contiguous.tile_stats(gi, scaler.loss_scale_factor)
            else:
                ptrs, tensors, grad_dtype = g.grad_pointers()
                keep.extend(tensors)
            lr, betas, eps, wd = FlatAdam.hyper(group)
            launches.append(GroupLaunch(
                group=g, lr=lr, betas=betas, eps=eps, weight_decay=wd,
                step=state["step"] + 1, exp_avg=state["exp_avg"], exp_avg_sq=state["exp_avg_sq"],
                grads=ptrs, grad_dtype=grad_dtype, tile_stats=tile_stats,
            ))

        def model_targets():
            # runs while K1 is on the device: release param.grad (flat.py:213)
            # and collect the cast targets
            for g in self.flat_groups:
                g.release_grads()
            return self._model_targets()

        scalars = run_boundary(
            launches, ws, scaler=scaler, max_norm=max_norm,
            materialize_flat_grad=materialize_flat_grad, model_targets=model_targets,
            timer=self.launch_timer, keep=keep,
        )
        del keep  # recorded on the boundary's stream by run_boundary
        overflow = bool(scalars.overflow)
        if not overflow:
            self.grad_norm = float(scalars.norm)
        self._after_boundary(overflow)
        return scalars

    def commit_step(self) -> None:
        """Advance every group's Adam step counter after an applied update
        (adam.py:86)."""
        for st in self.adam.state:
            st["step"] += 1

    # ---------------------------------------------------------- persistence
    def state_dict(self) -> dict:
        return self.adam.state_dict()

    def load_state_dict(self, state: dict) -> None:
        self.adam.load_state_dict(state)

