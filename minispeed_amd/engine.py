"""Training engine with minispeed's API (minispeed/engine.py).

    import minispeed_amd as ms
    engine, optimizer, _, lr_scheduler = ms.initialize(
        model=model, model_parameters=model.parameters(), config=ds_config)
    loss = engine(x, y)
    engine.backward(loss)
    engine.step()          # no-op until the accumulation boundary

Micro-batch bookkeeping, loss scaling in ``backward`` and the boundary
gating are host logic with the reference's semantics (engine.py:158-266).
At the boundary, ``_take_optimizer_step`` runs the whole
flatten / inf-nan / unscale / norm / clip / AdamW / cast sequence as three
HIP kernels with one device->host read-back, then applies the reference's
host bookkeeping (engine.py:268-322): on overflow the step is skipped, the
loss scale halves and neither the scheduler nor the Adam step advances; on
success ``grad_norm`` is set, the scale window advances and the scheduler
steps.
"""

from __future__ import annotations

import logging
from typing import Iterable, Iterator, List, Optional, Union

import torch
from torch import nn
from torch.utils._pytree import tree_map_only

from . import _native, comm
from . import checkpoint as ckpt
from .config import DeepSpeedConfig, load_config
from .contiguous import ContiguousGradients
from .flat import FlatParamGroup, build_flat_groups
from .flat import _walk as flat_walk
from .optim import build_scheduler
from .precision import DynamicLossScaler
from .utils import Timers
from .zero import build_zero_optimizer

logger = logging.getLogger("minispeed_amd")


def _normalize_param_groups(model: nn.Module, model_parameters, defaults: dict) -> List[dict]:
    """torch.optim-style groups, a flat iterable of params, a single group
    dict, or ``None`` (all model parameters) -> list of group dicts holding
    only trainable ``nn.Parameter``s, options merged over ``defaults``
    (engine.py:44-78)."""
    if model_parameters is None:
        raw = [list(model.parameters())]
    elif isinstance(model_parameters, dict):
        raw = [model_parameters]
    else:
        items = list(model_parameters)
        raw = items if items and isinstance(items[0], dict) else [items]
    groups = []
    for entry in raw:
        if isinstance(entry, dict):
            params = entry.get("params", [])
            opts = {k: v for k, v in entry.items() if k != "params"}
        else:
            params, opts = entry, {}
        merged = {**defaults, **opts}
        merged["params"] = [p for p in params if isinstance(p, nn.Parameter) and p.requires_grad]
        if merged["params"]:
            groups.append(merged)
    if not groups:
        raise ValueError("No trainable parameters found")
    return groups


class DeepSpeedEngine:
    """Wraps a ``torch.nn.Module``; fp32 masters in flat HBM buffers."""

    def __init__(self, model: nn.Module, config: Union[DeepSpeedConfig, dict, str, None], model_parameters=None):
        self.config = load_config(config, world_size=comm.get_world_size())
        self.rank = comm.get_rank()
        self.world_size = comm.get_world_size()
        self.device = comm.resolve_device()
        if self.device.type != "cuda":
            raise RuntimeError(
                f"device {self.device}: the boundary step runs as HIP kernels on a ROCm GPU"
            )
        # fail now, not at the first boundary, if a native part is missing
        _native.load()
        flat_walk()
        self.timers = Timers()
        self.module = model.to(self.device)

        groups = _normalize_param_groups(model, model_parameters, self.config.optimizer_params)
        self.flat_groups: List[FlatParamGroup]
        self.flat_groups, option_groups = build_flat_groups(
            groups, rank=self.rank, world_size=self.world_size,
            zero_stage=self.config.zero_stage, device=self.device,
            state_spacing=self.config.state_spacing_bytes,
        )
        # where the masters and moments were put (flat.place_state)
        self.state_placement = self.flat_groups[0].state_placement
        for g in self.flat_groups:
            g.copy_model_to_flat()

        self._param_dtype = None
        if self.config.dtype != "fp32":
            self._param_dtype = self.config.torch_dtype
            for g in self.flat_groups:
                for p in g.params:
                    p.data = p.data.to(self._param_dtype)

        if self.config.zero_stage >= 3:
            for g in self.flat_groups:
                g.partition_params()

        self.optimizer = build_zero_optimizer(self.flat_groups, option_groups, zero_stage=self.config.zero_stage)
        if self.config.zero_stage >= 3:
            self.optimizer.gather_reuse = self.config.stage3_gather_reuse
        self.contiguous: Optional[ContiguousGradients] = None
        if self.config.contiguous_gradients:
            self.contiguous = ContiguousGradients(
                self.flat_groups, scale_fn=lambda: self.loss_scaler.loss_scale_factor)
            self.optimizer.contiguous = self.contiguous
        self.lr_scheduler = build_scheduler(
            self.optimizer, self.config.scheduler_type, self.config.scheduler_params
        )
        self.loss_scaler = DynamicLossScaler(
            enabled=self.config.fp16_enabled,
            init_scale=self.config.loss_scale,
            scale_window=self.config.loss_scale_window,
        )
        if self.config.fp16_enabled and self.config.loss_scale == 0:
            self.loss_scaler.set_scale_from_power(self.config.initial_scale_power)

        self.micro_steps = 0
        self.global_steps = 0
        self._consumed_boundary = -1
        self.skipped_steps = 0
        self.grad_norm: Optional[float] = None
        self.last_boundary = None  # host copy of the last ms_step_scalars_t

    # ------------------------------------------------------------ properties
    @property
    def gas(self) -> int:
        return self.config.gas

    @property
    def is_gradient_accumulation_boundary(self) -> bool:
        return self.micro_steps > 0 and self.micro_steps % self.gas == 0

    @property
    def _boundary_pending(self) -> bool:
        return self.is_gradient_accumulation_boundary and self._consumed_boundary != self.micro_steps

    @property
    def loss_scale(self) -> float:
        return self.loss_scaler.loss_scale_factor

    @property
    def parameters(self) -> Iterable[nn.Parameter]:
        return self.module.parameters()

    # ------------------------------------------------------------ nn surface
    def _cast_inputs(self, obj):
        """Floating-point tensors anywhere in ``obj`` (nested lists, tuples,
        dicts) are cast to the model dtype; everything else passes through
        (engine.py:182-198)."""
        target = self._param_dtype
        if target is None:
            return obj

        def cast(t: torch.Tensor) -> torch.Tensor:
            return t.to(target) if t.is_floating_point() else t

        return tree_map_only(torch.Tensor, cast, obj)

    def forward(self, *args, **kwargs):
        if not self.optimizer.params_gathered:
            with self.timers.timer("gather"):
                self.optimizer.gather_parameters()
        return self.module(*self._cast_inputs(args), **self._cast_inputs(kwargs))

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)

    def train(self, mode: bool = True):
        self.module.train(mode)
        return self

    def eval(self):
        self.module.eval()
        return self

    def __iter__(self) -> Iterator:
        return iter((self, self.optimizer, None, self.lr_scheduler))

    # ------------------------------------------------------------- backward
    def _scale_loss(self, loss: torch.Tensor, scale_wrt_gas: bool) -> torch.Tensor:
        factor = self.loss_scaler.loss_scale_factor
        if scale_wrt_gas and self.gas > 1:
            factor /= self.gas
        return loss if factor == 1.0 else loss * factor

    def backward(self, loss: torch.Tensor, scale_wrt_gas: bool = True,
                 retain_graph: bool = False, create_graph: bool = False) -> None:
        """``loss * scale / gas`` then autograd; gradients accumulate on the
        parameters in the model dtype until the boundary (engine.py:235-251)."""
        with self.timers.timer("backward"):
            scaled = self._scale_loss(loss, scale_wrt_gas=scale_wrt_gas)
            scaled.backward(retain_graph=retain_graph, create_graph=create_graph)
        self.micro_steps += 1

    # ----------------------------------------------------------------- step
    def step(self) -> bool:
        """True only when an optimizer update was applied (engine.py:254-266)."""
        if not self._boundary_pending:
            return False
        self._consumed_boundary = self.micro_steps
        with self.timers.timer("step"):
            return self._take_optimizer_step()

    @torch.no_grad()
    def _take_optimizer_step(self) -> bool:
        scalars = self.optimizer.boundary_step(
            self.loss_scaler, self.config.gradient_clipping,
            materialize_flat_grad=self.config.materialize_flat_grad,
        )
        self.last_boundary = scalars
        if self.contiguous is not None:
            self.contiguous.next_window()
        overflow = bool(scalars.overflow)
        self._check_device_scaler(scalars, self.loss_scaler.expected(overflow))
        self.loss_scaler.update(overflow=overflow)
        if overflow:
            self.skipped_steps += 1
            self.optimizer.zero_grad()
            if self.skipped_steps % max(1, self.config.steps_per_print) == 0:
                logger.warning(
                    "rank %d: detected inf/nan gradients at micro_step=%d, skipping step "
                    "(loss_scale=%.1f, skipped=%d)",
                    self.rank, self.micro_steps, self.loss_scaler.scale, self.skipped_steps,
                )
            return False
        self.grad_norm = float(scalars.norm)
        self.optimizer.commit_step()
        self.lr_scheduler.step()
        self.optimizer.zero_grad()
        self.global_steps += 1
        return True

    def _check_device_scaler(self, scalars, expected) -> None:
        """K2 moved the loss-scale machine on the device; the host's
        transition of the same state (``precision.scale_transition``) must
        land on the same (scale, good_steps, skipped_steps)."""
        if not self.loss_scaler.enabled:
            return
        device = (scalars.next_scale, scalars.next_good_steps, scalars.next_skipped_steps)
        if device != tuple(expected):
            raise RuntimeError(
                f"device loss-scale decision {device} differs from the host scaler's {tuple(expected)}")

    def zero_grad(self, set_to_none: bool = True) -> None:
        if self.contiguous is not None:
            self.contiguous.next_window()
        for g in self.flat_groups:
            g.zero_grad()
        for p in self.module.parameters():
            p.grad = None

    # ---------------------------------------------------------- state dicts
    def state_dict(self):
        self.optimizer.gather_parameters()
        return self.module.state_dict()

    def load_state_dict(self, state_dict):
        self.optimizer.gather_parameters()
        self.module.load_state_dict(state_dict)
        # where the masters and moments were put (flat.place_state)
        self.state_placement = self.flat_groups[0].state_placement
        for g in self.flat_groups:
            g.copy_model_to_flat()

    def save_checkpoint(self, save_dir: str, tag: Optional[str] = None, **kwargs):
        """minispeed's checkpoint layout (checkpoint.py:35-71)."""
        return ckpt.save_checkpoint(self, save_dir, tag=tag)

    def load_checkpoint(self, load_dir: str, tag: Optional[str] = None, **kwargs):
        """Resume from a checkpoint in minispeed's layout (checkpoint.py:74-125)."""
        return ckpt.load_checkpoint(self, load_dir, tag=tag)

    def get_loss_scale(self) -> float:
        return self.loss_scaler.scale

    def get_gradient_norm(self) -> Optional[float]:
        return self.grad_norm

    def __repr__(self) -> str:  # pragma: no cover
        return (f"DeepSpeedEngine({self.config!r}, global_steps={self.global_steps}, "
                f"micro_steps={self.micro_steps})")


def initialize(model: Optional[nn.Module] = None, model_parameters=None,
               config: Union[DeepSpeedConfig, dict, str, None] = None, model_args=None):
    """Build the engine; it unpacks as ``engine, optimizer, _, lr_scheduler``
    (engine.py:372-389)."""
    if model is None:
        raise ValueError("model is required")
    comm.init_distributed()
    engine = DeepSpeedEngine(model, config, model_parameters=model_parameters)
    if comm.get_rank() == 0:
        logger.info("minispeed_amd initialized: %s", engine.config)
    return engine
