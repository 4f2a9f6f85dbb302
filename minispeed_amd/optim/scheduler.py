"""LR schedules with DeepSpeed's config schema (minispeed/optim/scheduler.py).

Host-side scalar math: each ``step()`` writes the new lr into every
``optimizer.param_groups[i]["lr"]``.  The engine steps the schedule after
every applied (non-skipped) optimizer step and never at construction
(``last_epoch`` starts at -1, scheduler.py:31), so the first optimizer step
uses the optimizer's own lr and step k >= 2 uses ``get_lr`` at epoch k-2.

    WarmupLR       lr(e) = min + (max-min) * e / warm   for e < warm, else max
    WarmupDecayLR  warmup as above, then
                   lr(e) = min + (max-min) * (total-e) / max(1, total-warm)
                   and min once e >= total            (scheduler.py:80-95)
"""

from __future__ import annotations

from typing import Optional


class _WarmupBase:
    def __init__(
        self,
        optimizer,
        warmup_min_lr: float = 0.0,
        warmup_max_lr: float = 1e-3,
        warmup_num_steps: int = 0,
        total_num_steps: Optional[int] = None,
    ):
        self.optimizer = optimizer
        self.warmup_min_lr = float(warmup_min_lr)
        self.warmup_max_lr = float(warmup_max_lr)
        self.warmup_num_steps = max(0, int(warmup_num_steps))
        self.total_num_steps = None if total_num_steps is None else int(total_num_steps)
        self.last_epoch = -1
        self.base_lrs = [float(g.get("lr", self.warmup_max_lr)) for g in optimizer.param_groups]

    def _warmup_lr(self, epoch: int) -> float:
        warm = self.warmup_num_steps
        if warm > 0 and epoch < warm:
            span = self.warmup_max_lr - self.warmup_min_lr
            return self.warmup_min_lr + span * (epoch / warm)
        return self.warmup_max_lr

    def get_lr(self) -> float:  # pragma: no cover - abstract
        raise NotImplementedError

    def step(self, epoch: Optional[int] = None) -> None:
        self.last_epoch = self.last_epoch + 1 if epoch is None else epoch
        lr = self.get_lr()
        for group in self.optimizer.param_groups:
            group["lr"] = lr

    def get_last_lr(self) -> float:
        return float(self.optimizer.param_groups[0]["lr"])

    def state_dict(self) -> dict:
        return {
            "type": type(self).__name__,
            "last_epoch": self.last_epoch,
            "warmup_min_lr": self.warmup_min_lr,
            "warmup_max_lr": self.warmup_max_lr,
            "warmup_num_steps": self.warmup_num_steps,
            "total_num_steps": self.total_num_steps,
        }

    def load_state_dict(self, state: dict) -> None:
        self.last_epoch = int(state["last_epoch"])


class WarmupLR(_WarmupBase):
    """Linear warmup to ``warmup_max_lr``, then constant."""

    def get_lr(self) -> float:
        return self._warmup_lr(self.last_epoch)


class WarmupDecayLR(_WarmupBase):
    """Linear warmup, then linear decay to ``warmup_min_lr`` at
    ``total_num_steps``."""

    def get_lr(self) -> float:
        e = self.last_epoch
        warm = self.warmup_num_steps
        if e < warm:
            return self._warmup_lr(e)
        total = self.total_num_steps
        if total is None:
            return self.warmup_max_lr
        if e >= total:
            return self.warmup_min_lr
        frac = (total - e) / max(1, total - warm)
        return self.warmup_min_lr + (self.warmup_max_lr - self.warmup_min_lr) * frac


class ConstantLR(WarmupLR):
    """Config alias of WarmupLR."""


_SCHEDULERS = {
    "WarmupLR": WarmupLR,
    "WarmupLRConst": WarmupLR,
    "ConstantLR": WarmupLR,
    "WarmupDecayLR": WarmupDecayLR,
}


def build_scheduler(optimizer, scheduler_type: str, params: dict):
    cls = _SCHEDULERS.get(scheduler_type)
    if cls is None:
        raise ValueError(f"Unknown scheduler type: {scheduler_type}")
    return cls(
        optimizer,
        warmup_min_lr=params.get("warmup_min_lr", 0.0),
        warmup_max_lr=params.get("warmup_max_lr"),
        warmup_num_steps=params.get("warmup_num_steps", 0),
        total_num_steps=params.get("total_num_steps"),
    )
