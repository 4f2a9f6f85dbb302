"""The engine on the GPU against minispeed's recorded trajectories.

Every golden case is replayed through ``ms.initialize`` / ``engine.step`` on
the GPU.  At each boundary the oracle is started from the GPU's own state
(masters, moments, step counters, scaler, schedule) and given the same
gradients, so each step is checked on its own:

* exact: step applied or skipped, loss-scale state, lr, Adam step counters,
  global step count; the model-dtype parameters equal the round-to-nearest-
  even cast of the GPU masters;
* grad_norm within 1e-5 relative, and the clip decision the reference's
  formula makes for the GPU's norm;
* with the oracle's AdamW run on the gradients the GPU clipped (the GPU's
  clip coefficient, ``clip_override``): exp_avg / exp_avg_sq bit-exact, and
  the masters' last rounding accounted for element by element
  (``tests/helpers.py:master_step_within_ulps``): the oracle's masters are
  the update recomputed from those moments with torch's CPU sqrt, the
  GPU's the same with a correctly rounded sqrt, bit for bit, and the two
  are within 2 fp32 ulp of the oracle's result wherever the sqrts agree.

The trajectory as a whole must also stay within 1e-5 relative of the
recorded one, element by element, relative to the element's largest
magnitude along the run.
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
from tests.helpers import clip_override, master_step_within_ulps, relative_within, step_hyper
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
    init_masters = [_cpu(g.data).numpy() for g in engine.flat_groups]

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
        hps = [step_hyper(engine, gi) for gi in range(len(engine.flat_groups))]
        applied = engine.step()
        assert applied == rec["applied"], step
        # the oracle's AdamW on the gradients the GPU clipped (same coefficient)
        assert ref.step(clip_override=clip_override(engine) if applied else None) == applied

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
            if clip is not None:    # the GPU's clip decision is the reference formula's
                applied_ref, _, _ = recipe.clip_coef(np.float32(engine.grad_norm), clip)
                assert bool(engine.last_boundary.clip_applied) == applied_ref

        for gi, (g, rg) in enumerate(zip(engine.flat_groups, ref.groups)):
            got_p = _cpu(g.data).numpy()
            want_p = rg.data.numpy()
            for got, want in ((engine.optimizer.state[gi]["exp_avg"], ref.state[gi]["exp_avg"]),
                              (engine.optimizer.state[gi]["exp_avg_sq"], ref.state[gi]["exp_avg_sq"])):
                np.testing.assert_array_equal(_cpu(got).numpy(), want.numpy())
            st = engine.optimizer.state[gi]
            if applied:
                ok, worst, nsq = master_step_within_ulps(before[gi].numpy(), got_p, want_p,
                                                         _cpu(st["exp_avg"]).numpy(),
                                                         _cpu(st["exp_avg_sq"]).numpy(), **hps[gi])
                assert ok, (step, gi, worst, nsq)
            else:            # a skipped step leaves the masters untouched
                np.testing.assert_array_equal(got_p.view(np.int32), before[gi].numpy().view(np.int32))
                np.testing.assert_array_equal(want_p.view(np.int32), got_p.view(np.int32))
            # against minispeed's recorded trajectory: 1e-5 relative per
            # element, relative to the element's magnitude along the run
            rec_p = arr[f"s{step}_master{gi}"]
            scale = np.maximum(np.maximum(np.abs(rec_p), np.abs(init_masters[gi])), np.abs(got_p))
            ok, worst = relative_within(got_p, rec_p, scale)
            assert ok, (step, gi, worst)
            # model copy == cast of the masters (placeholders at stage 3)
            master = g.data.detach().cpu()
            for (off, p), n in zip(g._offsets, g._numels):
                want = master[off - g.master_range[0]:off - g.master_range[0] + n].to(p.dtype)
                np.testing.assert_array_equal(bits_of(p.data), bits_of(want))
        if stage >= 3:
            assert not engine.optimizer.params_gathered
            assert all(fg.grad is None for fg in engine.flat_groups)
