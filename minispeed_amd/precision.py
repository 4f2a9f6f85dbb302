"""Mixed-precision state: dynamic loss scaling and the inf/nan test.

``DynamicLossScaler`` is host state with the semantics of
minispeed/precision.py:10-76: the scale starts at ``2**initial_scale_power``
(or a positive static ``loss_scale``, which stays dynamic), halves on an
overflowing step down to ``min_scale``, and doubles after ``scale_window``
consecutive clean steps up to ``max_scale``; disabled (fp32/bf16) it is a
no-op with scale 1.  The boundary kernel computes the same decision on the
device; the engine checks that both agree.
"""

from __future__ import annotations

import torch

from . import comm


class DynamicLossScaler:
    def __init__(
        self,
        enabled: bool = True,
        init_scale: float = 0.0,
        scale_window: int = 1000,
        min_scale: float = 1.0,
        max_scale: float = 2.0 ** 24,
    ):
        self.enabled = enabled
        self.min_scale = min_scale
        self.max_scale = max_scale
        self.scale_window = max(1, scale_window)
        if enabled and init_scale and init_scale > 0:
            self.scale = float(init_scale)
        else:
            # disabled: fixed at 1; enabled without a static value: the engine
            # sets 2**initial_scale_power right after construction
            self.scale = 1.0
        self.good_steps = 0
        self.skipped_steps = 0

    def set_scale_from_power(self, power: int) -> None:
        if self.enabled:
            self.scale = float(2.0 ** int(power))

    @property
    def loss_scale_factor(self) -> float:
        return self.scale if self.enabled else 1.0

    def update(self, overflow: bool) -> None:
        """Advance the state machine after one step attempt (precision.py:50-62)."""
        if not self.enabled:
            return
        if overflow:
            self.scale = max(self.scale / 2.0, self.min_scale)
            self.good_steps = 0
            self.skipped_steps += 1
            return
        self.good_steps += 1
        if self.good_steps >= self.scale_window and self.scale < self.max_scale:
            self.scale = min(self.scale * 2.0, self.max_scale)
            self.good_steps = 0

    def state_dict(self) -> dict:
        return {
            "enabled": self.enabled,
            "scale": self.scale,
            "good_steps": self.good_steps,
            "skipped_steps": self.skipped_steps,
        }

    def load_state_dict(self, state: dict) -> None:
        self.enabled = bool(state.get("enabled", self.enabled))
        self.scale = float(state.get("scale", self.scale))
        self.good_steps = int(state.get("good_steps", 0))
        self.skipped_steps = int(state.get("skipped_steps", 0))


def has_overflow(*grad_buffers: torch.Tensor) -> bool:
    """True if any element of any buffer is inf/nan (precision.py:79-87).

    Runs the ragged-grad scan kernel over each buffer on its HIP device (one
    host sync per buffer); buffers that are ``None`` or empty are skipped.
    """
    from .boundary import scan_nonfinite

    for buf in grad_buffers:
        if buf is None or buf.numel() == 0:
            continue
        if scan_nonfinite(buf):
            return True
    return False


def global_overflow(local_overflow: bool) -> bool:
    """OR of the local flag over data-parallel ranks (precision.py:90-92)."""
    return comm.all_reduce_flag(local_overflow)
