"""The oracle's contiguous-gradient path, pinned on the CPU.

* ``accumulate_fp32`` equals exact rational sums where those are
  representable, and rounds once per add otherwise (checked against fp64);
* a boundary given the flat fp32 gradients equals the reference boundary
  that flattens the same gradients from ``param.grad`` (the path the golden
  vectors pin), bit for bit, for every golden case.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch
from torch import nn

from oracle import boundary as ob
from tests.golden_cases import (DTYPES, META, TRAJECTORY_CASES, arrays, case_grads,
                                group_options, scheduler_params)


def test_accumulate_fp32_exact_dyadic_sums():
    g = torch.Generator().manual_seed(0)
    parts = [(torch.randint(-2048, 2048, (1000,), generator=g) / 64).to(torch.float16)
             for _ in range(5)]
    acc = None
    for x in parts:
        acc = ob.accumulate_fp32(acc, x)
    want = [sum(Fraction(float(x[i])) for x in parts) for i in range(1000)]
    assert [Fraction(float(v)) for v in acc] == want


def test_accumulate_fp32_rounds_once_per_add():
    g = torch.Generator().manual_seed(1)
    a = torch.randn(4096, generator=g).to(torch.bfloat16)
    b = (torch.randn(4096, generator=g) * 1e-3).to(torch.bfloat16)
    acc = ob.accumulate_fp32(ob.accumulate_fp32(None, a), b)
    want = (a.double() + b.double()).float()      # one rounding of the exact sum
    assert torch.equal(acc, want)
    assert acc.dtype == torch.float32
    inf = torch.tensor([float("inf"), 1.0], dtype=torch.float16)
    out = ob.accumulate_fp32(ob.accumulate_fp32(None, inf), torch.ones(2, dtype=torch.float16))
    assert torch.isinf(out[0]) and out[1] == 2.0


def _engine(case, arr):
    cfg = case["config"]
    params = [nn.Parameter(torch.from_numpy(arr[f"init_p{i}"].copy()))
              for i in range(len(case["shapes"]))]
    fp16 = cfg.get("fp16", {})
    clip = cfg.get("gradient_clipping")
    eng = ob.Engine([[params[i] for i in idx] for idx in case["groups"]], group_options(case),
                    dtype=cfg["dtype"], zero_stage=cfg["zero_optimization"]["stage"],
                    clip=float(clip) if clip else None,
                    loss_scale=float(fp16.get("loss_scale", 0.0)),
                    initial_scale_power=int(fp16.get("initial_scale_power", 16)),
                    loss_scale_window=int(fp16.get("loss_scale_window", 1000)),
                    scheduler=cfg["scheduler"]["type"], scheduler_params=scheduler_params(cfg))
    return eng, params


@pytest.mark.parametrize("name", TRAJECTORY_CASES)
def test_boundary_from_flat_grads_equals_the_flatten_path(name):
    case = META["cases"][name]
    arr = arrays(name)
    dtype = DTYPES[case["config"]["dtype"]]
    stage = case["config"]["zero_optimization"]["stage"]
    a, pa = _engine(case, arr)
    b, pb = _engine(case, arr)
    for step in range(case["steps"]):
        if stage >= 3:
            a.gather_parameters()
            b.gather_parameters()
        grads = case_grads(case, arr, step, dtype)
        for p, g in zip(pa, grads):
            p.grad = None if g is None else g.clone()
        flats = []
        for grp, idx in zip(b.groups, case["groups"]):
            f = torch.zeros(grp.numel_padded, dtype=torch.float32)
            for off, i in zip(grp.offsets, idx):
                if grads[i] is not None:
                    f[off:off + grads[i].numel()] = ob.accumulate_fp32(None, grads[i])
            flats.append(f)
        a.micro_steps += 1
        b.micro_steps += 1
        assert a.step() == b.step(flat_grads=flats)
        assert a.grad_norm == b.grad_norm and a.scaler.scale == b.scaler.scale
        for ga, gb in zip(a.groups, b.groups):
            assert torch.equal(ga.data, gb.data)
        for sa, sb in zip(a.state, b.state):
            assert torch.equal(sa["exp_avg"], sb["exp_avg"])
            assert torch.equal(sa["exp_avg_sq"], sb["exp_avg_sq"])
