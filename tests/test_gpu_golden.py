"""The engine on the GPU against minispeed's recorded trajectories.

Every golden case is replayed through ``ms.initialize`` / ``engine.step`` on
the GPU.  At each boundary the oracle is started from the GPU's own state
(masters, moments, step counters, scaler, schedule) and given the same
gradients, so each step is checked on its own:

* exact: step applied or skipped, loss-scale state, lr, Adam step counters,
  global step count; the model-dtype parameters equal the round-to-nearest-
  even cast of the GPU masters;
* grad_norm within 1e-5 relative;
* exp_avg / exp_avg_sq bit-exact whenever both sides used the same fp32
  clip coefficient (within 1e-6 relative otherwise);
* masters within 2 fp32 ulp per step, in units of the largest operand of
  the final addition p + u (max of |p_before|, |u|, |p_after|).

The trajectory as a whole must also stay within 1e-5 relative of the
recorded one.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch
from torch import nn

import minispeed_amd as ms
from oracle import boundary as ob
from oracle import recipe
from tests.helpers import master_step_within_ulps
from tests.golden_cases import (DTYPES, META, TRAJECTORY_CASES, arrays, bits_of, case_grads,
                                group_options, scheduler_params)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _oracle(case, arr):
    cfg = case["config"]
    shapes = case["shapes"]
    params = [nn.Parameter(torch.from_numpy(arr[f"init_p{i}"].copy())) for i in range(len(shapes))]
    groups = [[params[i] for i in idx] for idx in case["groups"]]
    fp16 = cfg.get("fp16", {})
    clip = cfg.get("gradient_clipping")
    eng = ob.Engine(groups, group_options(case), dtype=cfg["dtype"],
                    zero_stage=cfg["zero_optimization"]["stage"],
                    clip=float(clip) if clip else None,
                    loss_scale=float(fp16.get("loss_scale", 0.0)),
                    initial_scale_power=int(fp16.get("initial_scale_power", 16)),
                    loss_scale_window=int(fp16.get("loss_scale_window", 1000)),
                    scheduler=cfg["scheduler"]["type"], scheduler_params=scheduler_params(cfg))
    return eng, params


def _engine(case, arr):
    shapes = case["shapes"]
    params = [nn.Parameter(torch.from_numpy(arr[f"init_p{i}"].copy()).to(DEV))
              for i in range(len(shapes))]
    module = nn.ParameterList(params)
    extra = case.get("group_opts") or []
    if len(case["groups"]) == 1 and not extra:
        mp = [params[i] for i in case["groups"][0]]
    else:
        mp = []
        for k, idx in enumerate(case["groups"]):
            d = {"params": [params[i] for i in idx]}
            for key, v in (extra[k] if extra else {}).items():
                d[key] = tuple(v) if key == "betas" else v
            mp.append(d)
    engine = ms.initialize(model=module, model_parameters=mp, config=copy.deepcopy(case["config"]))
    return engine, params


def _cpu(t):
    return t.detach().float().cpu().clone()


@pytest.mark.parametrize("name", TRAJECTORY_CASES)
def test_engine_replays_golden_case(name):
    case = META["cases"][name]
    arr = arrays(name)
    cfg = case["config"]
    stage = cfg["zero_optimization"]["stage"]
    dtype = DTYPES[cfg["dtype"]]
    clip = cfg.get("gradient_clipping")
    clip = float(clip) if clip else None
    engine, params = _engine(case, arr)
    ref, ref_params = _oracle(case, arr)
    assert len(engine.flat_groups) == len(ref.groups)

    for step, rec in enumerate(case["trajectory"]):
        before = [_cpu(g.data) for g in engine.flat_groups]
        ref.load_state(
            before, [_cpu(st["exp_avg"]) for st in engine.optimizer.state],
            [_cpu(st["exp_avg_sq"]) for st in engine.optimizer.state],
            [st["step"] for st in engine.optimizer.state],
            (engine.loss_scaler.scale, engine.loss_scaler.good_steps, engine.loss_scaler.skipped_steps),
            engine.lr_scheduler.last_epoch, [g["lr"] for g in engine.optimizer.param_groups])
        if stage >= 3:
            engine.optimizer.gather_parameters()
            ref.gather_parameters()
        for p, rp, g in zip(params, ref_params, case_grads(case, arr, step, dtype)):
            p.grad = None if g is None else g.to(DEV)
            rp.grad = None if g is None else g.clone()
        engine.micro_steps += 1
        ref.micro_steps += 1
        applied = engine.step()
        assert applied == ref.step() == rec["applied"], step

        s = engine.loss_scaler
        assert (s.scale, s.good_steps, s.skipped_steps) == (rec["scale"], rec["good_steps"],
                                                            rec["skipped_steps"])
        assert [g["lr"] for g in engine.optimizer.param_groups] == rec["lr"]
        assert [st["step"] for st in engine.optimizer.state] == rec["adam_step"]
        assert engine.global_steps == rec["global_steps"]
        if rec["grad_norm"] is None:
            assert engine.grad_norm is None
        else:
            assert abs(engine.grad_norm - rec["grad_norm"]) <= 1e-5 * rec["grad_norm"]
        if applied:
            assert abs(engine.grad_norm - ref.grad_norm) <= 1e-5 * ref.grad_norm
        same_coef = True
        if applied and clip is not None:
            _, _, ref_coef = recipe.clip_coef(np.float32(ref.grad_norm), clip)
            same_coef = np.float32(engine.last_boundary.coef) == np.float32(ref_coef)

        for gi, (g, rg) in enumerate(zip(engine.flat_groups, ref.groups)):
            got_p = _cpu(g.data).numpy()
            want_p = rg.data.numpy()
            for got, want in ((engine.optimizer.state[gi]["exp_avg"], ref.state[gi]["exp_avg"]),
                              (engine.optimizer.state[gi]["exp_avg_sq"], ref.state[gi]["exp_avg_sq"])):
                got = _cpu(got).numpy()
                if same_coef:
                    np.testing.assert_array_equal(got, want.numpy())
                else:
                    np.testing.assert_allclose(got, want.numpy(), rtol=1e-6,
                                               atol=1e-6 * float(np.abs(want.numpy()).max() or 1))
            ok, worst = master_step_within_ulps(before[gi].numpy(), got_p, want_p,
                                                2.0 if same_coef else 4.0)
            assert ok, (step, gi, worst)
            # against the recorded trajectory
            np.testing.assert_allclose(got_p, arr[f"s{step}_master{gi}"], rtol=1e-5,
                                       atol=1e-5 * float(np.abs(arr[f"s{step}_master{gi}"]).max()))
            # model copy == cast of the masters (placeholders at stage 3)
            master = g.data.detach().cpu()
            for (off, p), n in zip(g._offsets, g._numels):
                want = master[off - g.master_range[0]:off - g.master_range[0] + n].to(p.dtype)
                np.testing.assert_array_equal(bits_of(p.data), bits_of(want))
        if stage >= 3:
            assert not engine.optimizer.params_gathered
            assert all(fg.grad is None for fg in engine.flat_groups)
