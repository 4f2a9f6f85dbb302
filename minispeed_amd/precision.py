"""Mixed-precision state: the dynamic loss scale and the inf/nan test.

The loss scale is a small state machine over ``(scale, good_steps,
skipped_steps)`` with minispeed's semantics (precision.py:10-76):

* an overflowing step halves the scale (never below ``min_scale``), clears
  the run of clean steps and counts one skipped step;
* a clean step extends the run; once the run reaches ``scale_window`` and
  the scale is below ``max_scale`` the scale doubles (capped at
  ``max_scale``) and the run starts over;
* disabled (fp32 / bf16) the machine never moves and the scale is 1.

``scale_transition`` is that machine as a pure function.  The boundary
kernel makes the same decision on the device (K2 writes the next state next
to the norm); the engine computes the host's expectation with this function
and refuses to continue if the two differ.  ``DynamicLossScaler`` is the
stateful object the engine and checkpoints use, a thin holder of one
``ScaleState``.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from . import comm


class ScaleState(NamedTuple):
    scale: float
    good_steps: int
    skipped_steps: int


def scale_transition(state: ScaleState, overflow: bool, *, window: int,
                     min_scale: float, max_scale: float) -> ScaleState:
    """The state after one step attempt (precision.py:50-62)."""
    scale, good, skipped = state
    if overflow:
        return ScaleState(max(scale / 2.0, min_scale), 0, skipped + 1)
    good += 1
    if good < window or not scale < max_scale:
        return ScaleState(scale, good, skipped)
    return ScaleState(min(scale * 2.0, max_scale), 0, skipped)


class DynamicLossScaler:
    """Loss-scale state of one engine.

    ``init_scale > 0`` starts the enabled machine at that value (it stays
    dynamic); otherwise it starts at 1 and the engine applies
    ``initial_scale_power`` through :meth:`set_scale_from_power`.
    """

    def __init__(self, enabled: bool = True, init_scale: float = 0.0, scale_window: int = 1000,
                 min_scale: float = 1.0, max_scale: float = 2.0 ** 24):
        self.enabled = enabled
        self.min_scale = min_scale
        self.max_scale = max_scale
        self.scale_window = scale_window if scale_window > 1 else 1
        start = float(init_scale) if enabled and init_scale and init_scale > 0 else 1.0
        self._state = ScaleState(start, 0, 0)

    # the three fields of the state, readable and assignable one by one
    scale = property(lambda self: self._state.scale,
                     lambda self, v: self._set(scale=float(v)))
    good_steps = property(lambda self: self._state.good_steps,
                          lambda self, v: self._set(good_steps=int(v)))
    skipped_steps = property(lambda self: self._state.skipped_steps,
                             lambda self, v: self._set(skipped_steps=int(v)))

    def _set(self, **fields) -> None:
        self._state = self._state._replace(**fields)

    @property
    def state(self) -> ScaleState:
        return self._state

    def set_scale_from_power(self, power: int) -> None:
        if self.enabled:
            self._set(scale=float(2.0 ** int(power)))

    @property
    def loss_scale_factor(self) -> float:
        """What the loss is multiplied by in backward (1 when disabled)."""
        return self._state.scale if self.enabled else 1.0

    def expected(self, overflow: bool) -> ScaleState:
        """The state :meth:`update` would move to, without moving."""
        if not self.enabled:
            return self._state
        return scale_transition(self._state, overflow, window=self.scale_window,
                                min_scale=self.min_scale, max_scale=self.max_scale)

    def update(self, overflow: bool) -> None:
        self._state = self.expected(overflow)

    def state_dict(self) -> dict:
        return {"enabled": self.enabled, **self._state._asdict()}

    def load_state_dict(self, state: dict) -> None:
        """Fields missing from ``state`` keep the current ``enabled`` and
        ``scale`` and reset both counters to 0."""
        merged = {"enabled": self.enabled, "scale": self._state.scale,
                  "good_steps": 0, "skipped_steps": 0}
        merged.update(state)
        self.enabled = bool(merged["enabled"])
        self._state = ScaleState(float(merged["scale"]), int(merged["good_steps"]),
                                 int(merged["skipped_steps"]))


def has_overflow(*grad_buffers: torch.Tensor) -> bool:
    """True if any element of any buffer is inf/nan (precision.py:79-87).

    Runs the ragged-grad scan kernel over each buffer on its HIP device (one
    host sync per buffer); buffers that are ``None`` or empty are skipped.
    """
    from .boundary import scan_nonfinite

    return any(scan_nonfinite(buf) for buf in grad_buffers if buf is not None and buf.numel())


def global_overflow(local_overflow: bool) -> bool:
    """OR of the local flag over data-parallel ranks (precision.py:90-92)."""
    return comm.all_reduce_flag(local_overflow)
