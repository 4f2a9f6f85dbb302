"""LR schedules with DeepSpeed's config schema (minispeed/optim/scheduler.py).

A schedule is a pure function of an epoch counter and four numbers
(:class:`WarmupSpec`); the scheduler object only keeps the counter and
writes the function's value into every ``optimizer.param_groups[i]["lr"]``.

    warmup        lr(e) = lo + (hi - lo) * (e / warm)            e < warm
                  lr(e) = hi                                     otherwise
    warmup+decay  the warmup above while e < warm, then
                  lr(e) = lo + (hi - lo) * ((total - e) / max(1, total - warm))
                  and lo once e >= total                  (scheduler.py:37-95)

with lo, hi = ``warmup_min_lr``, ``warmup_max_lr``.  Both ramps are written
as ``lo + (hi - lo) * fraction`` with the fraction taken first, the order
whose double roundings the reference produces, so the per-step lr (and
hence the fp32 scalars of the AdamW kernel) match it exactly.

The engine advances the counter after every applied optimizer step and
never at construction (the counter starts at -1, scheduler.py:31): the
first update runs at the optimizer's own lr, update k >= 2 at lr(k - 2).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Dict, Optional


@dataclass(frozen=True)
class WarmupSpec:
    lo: float                  # warmup_min_lr
    hi: float                  # warmup_max_lr
    warm: int                  # warmup_num_steps (negative values act as 0)
    total: Optional[int]       # total_num_steps (decay only)


def _ramp(lo: float, hi: float, num: float, den: float) -> float:
    return lo + (hi - lo) * (num / den)


def warmup_lr(spec: WarmupSpec, epoch: int) -> float:
    if spec.warm > 0 and epoch < spec.warm:
        return _ramp(spec.lo, spec.hi, epoch, spec.warm)
    return spec.hi


def warmup_decay_lr(spec: WarmupSpec, epoch: int) -> float:
    if epoch < spec.warm:
        return warmup_lr(spec, epoch)
    if spec.total is None:
        return spec.hi
    if epoch >= spec.total:
        return spec.lo
    return _ramp(spec.lo, spec.hi, spec.total - epoch, max(1, spec.total - spec.warm))


class _Scheduled:
    """Epoch counter + one schedule function (``shape``)."""

    shape: Callable[[WarmupSpec, int], float] = staticmethod(warmup_lr)

    def __init__(self, optimizer, warmup_min_lr: float = 0.0, warmup_max_lr: float = 1e-3,
                 warmup_num_steps: int = 0, total_num_steps: Optional[int] = None):
        self.optimizer = optimizer
        self.spec = WarmupSpec(float(warmup_min_lr), float(warmup_max_lr),
                               max(0, int(warmup_num_steps)),
                               None if total_num_steps is None else int(total_num_steps))
        self.base_lrs = [float(g.get("lr", self.spec.hi)) for g in optimizer.param_groups]
        self.last_epoch = -1

    # the config values under their schema names
    warmup_min_lr = property(lambda self: self.spec.lo)
    warmup_max_lr = property(lambda self: self.spec.hi)
    warmup_num_steps = property(lambda self: self.spec.warm)
    total_num_steps = property(lambda self: self.spec.total)

    def get_lr(self) -> float:
        return self.shape(self.spec, self.last_epoch)

    def step(self, epoch: Optional[int] = None) -> None:
        self.last_epoch = self.last_epoch + 1 if epoch is None else epoch
        lr = self.get_lr()
        for group in self.optimizer.param_groups:
            group["lr"] = lr

    def get_last_lr(self) -> float:
        return float(self.optimizer.param_groups[0]["lr"])

    def state_dict(self) -> dict:
        keys = ("warmup_min_lr", "warmup_max_lr", "warmup_num_steps", "total_num_steps")
        return {"type": type(self).__name__, "last_epoch": self.last_epoch,
                **dict(zip(keys, (self.spec.lo, self.spec.hi, self.spec.warm, self.spec.total)))}

    def load_state_dict(self, state: dict) -> None:
        """Only the counter is restored; the schedule comes from the config."""
        self.last_epoch = int(state["last_epoch"])


class WarmupLR(_Scheduled):
    """Linear warmup to ``warmup_max_lr``, then constant."""

    shape = staticmethod(warmup_lr)


class WarmupDecayLR(_Scheduled):
    """Linear warmup, then linear decay to ``warmup_min_lr`` at
    ``total_num_steps``."""

    shape = staticmethod(warmup_decay_lr)


class ConstantLR(WarmupLR):
    """Config alias of WarmupLR."""


# config "type" -> class; the aliases build a WarmupLR (scheduler.py:102-114)
_BY_TYPE: Dict[str, type] = {
    "WarmupLR": WarmupLR,
    "WarmupLRConst": WarmupLR,
    "ConstantLR": WarmupLR,
    "WarmupDecayLR": WarmupDecayLR,
}


def build_scheduler(optimizer, scheduler_type: str, params: dict):
    try:
        cls = _BY_TYPE[scheduler_type]
    except KeyError:
        raise ValueError(f"Unknown scheduler type: {scheduler_type}") from None
    return cls(optimizer,
               warmup_min_lr=params.get("warmup_min_lr", 0.0),
               warmup_max_lr=params.get("warmup_max_lr"),
               warmup_num_steps=params.get("warmup_num_steps", 0),
               total_num_steps=params.get("total_num_steps"))
