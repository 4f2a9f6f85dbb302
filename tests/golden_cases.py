"""Readers of the golden fixtures written by tests/golden/make_golden.py."""

from __future__ import annotations

import json
import os
from typing import Dict, List

import numpy as np
import torch
from torch import nn

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

with open(os.path.join(GOLDEN_DIR, "cases.json"), "r", encoding="utf-8") as _fh:
    META = json.load(_fh)

TRAJECTORY_CASES = sorted(k for k, v in META["cases"].items() if "trajectory" in v)
TRACE_CASES = sorted(k for k, v in META["cases"].items() if "losses" in v)

DTYPES = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}


def arrays(name: str) -> Dict[str, np.ndarray]:
    with np.load(os.path.join(GOLDEN_DIR, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def from_bits(raw: np.ndarray, dtype: torch.dtype, shape) -> torch.Tensor:
    t = torch.from_numpy(raw.copy())
    if dtype in (torch.float16, torch.bfloat16):
        return t.view(dtype).reshape(shape)
    return t.view(torch.float32).reshape(shape)


def bits_of(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous().reshape(-1)
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy()
    return t.view(torch.int32).numpy()


def group_options(case: dict) -> List[dict]:
    """Per-group optimizer options as the reference engine merges them
    (config defaults, then the group's own keys)."""
    cfg = case["config"]
    base = dict(cfg["optimizer"]["params"])
    base["betas"] = tuple(float(b) for b in base["betas"])
    opts = []
    extra = case.get("group_opts") or [{} for _ in case["groups"]]
    for e in extra:
        d = dict(base)
        for k, v in e.items():
            d[k] = tuple(v) if k == "betas" else v
        opts.append(d)
    return opts


def scheduler_params(cfg: dict) -> dict:
    sp = dict(cfg["scheduler"]["params"])
    sp.setdefault("warmup_num_steps", 0)
    sp.setdefault("warmup_max_lr", float(cfg["optimizer"]["params"]["lr"]))
    sp.setdefault("warmup_min_lr", 0.0)
    return sp


def case_grads(case: dict, arr: dict, step: int, dtype: torch.dtype):
    """Gradients of one boundary: list of tensors (None: no gradient)."""
    out = []
    for i, shape in enumerate(case["shapes"]):
        if f"s{step}_g{i}_none" in arr:
            out.append(None)
        else:
            out.append(from_bits(arr[f"s{step}_g{i}"], dtype, shape))
    return out


class MLP(nn.Module):
    """The 8 -> 32 -> 32 -> 1 MLP of minispeed's tests/common.py:19-32."""

    def __init__(self):
        super().__init__()
        self.net = nn.Sequential(nn.Linear(8, 32), nn.Tanh(), nn.Linear(32, 32), nn.ReLU(),
                                 nn.LayerNorm(32), nn.Linear(32, 1))

    def forward(self, x):
        return self.net(x)


class Holder(nn.Module):
    """The module of the recorded cases: a ParameterList named ``ps``, so
    state-dict keys are ``ps.0`` ... ``ps.4`` (tests/golden/make_golden.py)."""

    def __init__(self, params):
        super().__init__()
        self.ps = nn.ParameterList(params)


CHECKPOINT_CASES = sorted(k for k, v in META["cases"].items() if "checkpoint" in v)


def checkpoint_root(name: str) -> str:
    """Directory of the checkpoint minispeed wrote part-way through a case."""
    return os.path.join(GOLDEN_DIR, "ckpt", name)
