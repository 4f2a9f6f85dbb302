"""AdamW state over flat fp32 groups (minispeed/optim/adam.py).

``FlatAdam`` owns the torch-style ``param_groups`` (lr, betas, eps,
weight_decay; schedulers write ``lr``) and, per group, ``step`` plus the
fp32 moments ``exp_avg`` / ``exp_avg_sq`` over the owned shard
(adam.py:38-65).  The update itself is the fused AdamW kernel; "Adam" and
"AdamW" both use decoupled weight decay (the reference never branches on
the optimizer type).
"""

from __future__ import annotations

import ctypes
from typing import List

import numpy as np
import torch

from .. import _native
from ..flat import FlatParamGroup

_DEFAULTS = {"lr": 1e-3, "betas": (0.9, 0.999), "eps": 1e-8, "weight_decay": 0.0}


class FlatAdam:
    def __init__(self, flat_groups: List[FlatParamGroup], option_groups: List[dict], zero_stage: int = 0):
        self.flat_groups = flat_groups
        self.zero_stage = zero_stage
        self.param_groups: List[dict] = []
        self._state: List[dict] = []
        for flat, opts in zip(flat_groups, option_groups):
            group = dict(opts)
            for key, value in _DEFAULTS.items():
                group.setdefault(key, value)
            self.param_groups.append(group)
            n = flat.numel_shard()
            moments = flat.take_moment_buffers()
            if moments is None or any(t.numel() != n for t in moments):
                moments = tuple(torch.zeros(n, dtype=torch.float32, device=flat.device) for _ in range(2))
            self._state.append({"step": 0, "exp_avg": moments[0], "exp_avg_sq": moments[1]})
        self._clean = None  # device "no overflow, no clip" scalars for step()

    @staticmethod
    def hyper(group: dict):
        """(lr, betas, eps, weight_decay) as the reference reads them
        (adam.py:72-75)."""
        lr = float(group["lr"])
        b1, b2 = group["betas"]
        return lr, (float(b1), float(b2)), float(group["eps"]), float(group.get("weight_decay", 0.0))

    @torch.no_grad()
    def step(self) -> bool:
        """Standalone AdamW over ``grad_for_shard()`` of every group (already
        reduced, unscaled and clipped), as optim/adam.py:59-93; the model
        parameters are not touched (``sync_parameters`` does that)."""
        from ..boundary import adamw_params

        lib = _native.load()
        for group, flat, state in zip(self.param_groups, self.flat_groups, self._state):
            shard = flat.shard
            grad = flat.grad_for_shard()
            if grad.shape != shard.shape:
                raise RuntimeError(f"grad/shard shape mismatch: {grad.shape} vs {shard.shape}")
            if self._clean is None or self._clean.device != flat.device:
                self._clean = torch.zeros(_native.SCALARS_BYTES, dtype=torch.uint8, device=flat.device)
            state["step"] += 1
            lr, betas, eps, wd = self.hyper(group)
            hp = adamw_params(lr, betas, eps, wd, state["step"])
            lo, hi = flat.own_range
            if hi <= lo:
                continue
            ptr, nseg = flat.table("adam_only").upload(np.array([[lo, hi - lo, 0, 0]], dtype=np.int64))
            rc = lib.ms_fused_adamw(
                shard.data_ptr(), state["exp_avg"].data_ptr(), state["exp_avg_sq"].data_ptr(),
                grad.data_ptr(), ptr, nseg, _native.DTYPE_F32, _native.DTYPE_F32, lo, hi,
                ctypes.byref(hp), self._clean.data_ptr(), _native.stream_handle(flat.device),
            )
            _native.check(rc, "ms_fused_adamw")
            flat.masters_written()
        return True

    def zero_grad(self) -> None:
        for flat in self.flat_groups:
            flat.zero_grad()

    def state_dict(self) -> dict:
        return {
            "param_groups": [dict(g) for g in self.param_groups],
            "shard_state": [
                {"step": st["step"], "exp_avg": st["exp_avg"].clone(), "exp_avg_sq": st["exp_avg_sq"].clone()}
                for st in self._state
            ],
        }

    def load_state_dict(self, state_dict: dict) -> None:
        for saved, group in zip(state_dict["param_groups"], self.param_groups):
            group.update({k: v for k, v in saved.items() if k != "params"})
        for saved, st in zip(state_dict["shard_state"], self._state):
            st["step"] = int(saved["step"])
            st["exp_avg"].copy_(saved["exp_avg"])
            st["exp_avg_sq"].copy_(saved["exp_avg_sq"])

    @property
    def state(self) -> List[dict]:
        return self._state
