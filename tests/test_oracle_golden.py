"""The oracle reproduces minispeed's own outputs bit for bit.

The fixtures were written by running minispeed itself on its CPU path
(tests/golden/make_golden.py): every boundary's inputs (initial parameters,
raw gradient bits, inf/nan injections, parameters without gradient) and
outputs (step applied or skipped, grad_norm, loss-scale state, lr, Adam step
counters, fp32 masters, exp_avg, exp_avg_sq, model-dtype parameter bits).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch import nn

from oracle import boundary as ob
from tests.golden_cases import (DTYPES, META, MLP, TRACE_CASES, TRAJECTORY_CASES, arrays,
                                bits_of, case_grads, from_bits, group_options,
                                scheduler_params)


def _oracle_engine(case, arr):
    cfg = case["config"]
    shapes = case["shapes"]
    params = [nn.Parameter(torch.from_numpy(arr[f"init_p{i}"].copy())) for i in range(len(shapes))]
    groups = [[params[i] for i in idx] for idx in case["groups"]]
    fp16 = cfg.get("fp16", {})
    clip = cfg.get("gradient_clipping")
    eng = ob.Engine(
        groups, group_options(case), dtype=cfg["dtype"],
        zero_stage=cfg["zero_optimization"]["stage"], clip=float(clip) if clip else None,
        gas=cfg.get("gradient_accumulation_steps", 1),
        loss_scale=float(fp16.get("loss_scale", 0.0)),
        initial_scale_power=int(fp16.get("initial_scale_power", 16)),
        loss_scale_window=int(fp16.get("loss_scale_window", 1000)),
        scheduler=cfg["scheduler"]["type"], scheduler_params=scheduler_params(cfg),
    )
    return eng, params


@pytest.mark.parametrize("name", TRAJECTORY_CASES)
def test_oracle_matches_reference_trajectory(name):
    case = META["cases"][name]
    arr = arrays(name)
    eng, params = _oracle_engine(case, arr)
    dtype = DTYPES[case["config"]["dtype"]]
    stage = case["config"]["zero_optimization"]["stage"]
    for step, rec in enumerate(case["trajectory"]):
        if stage >= 3:
            eng.gather_parameters()
        for p, g in zip(params, case_grads(case, arr, step, dtype)):
            p.grad = g
        eng.micro_steps += 1
        assert eng.step() == rec["applied"], step
        assert eng.grad_norm == rec["grad_norm"]
        s = eng.scaler
        assert (s.scale, s.good_steps, s.skipped_steps) == (rec["scale"], rec["good_steps"],
                                                            rec["skipped_steps"])
        assert [g["lr"] for g in eng.param_groups] == rec["lr"]
        assert [st["step"] for st in eng.state] == rec["adam_step"]
        assert eng.global_steps == rec["global_steps"]
        for gi, g in enumerate(eng.groups):
            np.testing.assert_array_equal(g.data.numpy(), arr[f"s{step}_master{gi}"])
            np.testing.assert_array_equal(eng.state[gi]["exp_avg"].numpy(), arr[f"s{step}_m{gi}"])
            np.testing.assert_array_equal(eng.state[gi]["exp_avg_sq"].numpy(), arr[f"s{step}_v{gi}"])
        for i, p in enumerate(params):
            np.testing.assert_array_equal(bits_of(p.data), arr[f"s{step}_model{i}"])


@pytest.mark.parametrize("name", TRACE_CASES)
def test_oracle_matches_reference_mlp_trace(name):
    case = META["cases"][name]
    arr = arrays(name)
    cfg = case["config"]
    threads = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        model = MLP()
        with torch.no_grad():
            for i, p in enumerate(model.parameters()):
                p.copy_(torch.from_numpy(arr[f"init_p{i}"]))
        opts = dict(cfg["optimizer"]["params"])
        opts["betas"] = tuple(opts["betas"])
        fp16 = cfg.get("fp16", {})
        eng = ob.Engine([list(model.parameters())], [opts], dtype=cfg["dtype"], zero_stage=0,
                        clip=cfg["gradient_clipping"], gas=case["gas"],
                        loss_scale=float(fp16.get("loss_scale", 0.0)),
                        initial_scale_power=int(fp16.get("initial_scale_power", 16)),
                        loss_scale_window=int(fp16.get("loss_scale_window", 1000)),
                        scheduler=cfg["scheduler"]["type"], scheduler_params=scheduler_params(cfg))
        x = torch.from_numpy(arr["x"])
        y = torch.from_numpy(arr["y"])
        dt = DTYPES[cfg["dtype"]]
        losses, boundaries = [], []
        for s in range(case["steps"]):
            for mi in range(case["gas"]):
                xb = x[s, mi] if dt == torch.float32 else x[s, mi].to(dt)   # engine.py:182-198
                loss = F.mse_loss(model(xb).float(), y[s, mi].float())
                losses.append(float(loss.detach()))
                eng.backward(loss)
                applied = eng.step()
                if eng.micro_steps % eng.gas == 0:
                    sc = eng.scaler
                    boundaries.append({"applied": bool(applied), "scale": sc.scale,
                                       "good_steps": sc.good_steps, "skipped_steps": sc.skipped_steps,
                                       "grad_norm": eng.grad_norm,
                                       "lr": [g["lr"] for g in eng.param_groups],
                                       "global_steps": eng.global_steps})
    finally:
        torch.set_num_threads(threads)
    assert losses == case["losses"]
    assert boundaries == case["boundaries"]
    assert eng.grad_norm == case["grad_norm"]
    assert eng.global_steps == case["global_steps"]
    for i, p in enumerate(model.parameters()):
        np.testing.assert_array_equal(bits_of(p.data), arr[f"final_p{i}"])
    np.testing.assert_array_equal(eng.groups[0].data.numpy(), arr["final_master0"])


def test_fixtures_cover_the_hot_path_cases():
    """The fixture set exercises every branch the boundary step has."""
    trajs = [META["cases"][n]["trajectory"] for n in TRAJECTORY_CASES]
    flat = [r for t in trajs for r in t]
    assert any(not r["applied"] for r in flat)                       # skip
    assert any(r["applied"] for r in flat)
    stages = {META["cases"][n]["config"]["zero_optimization"]["stage"] for n in TRAJECTORY_CASES}
    assert stages == {0, 1, 2, 3}
    dtypes = {META["cases"][n]["config"]["dtype"] for n in TRAJECTORY_CASES}
    assert dtypes == {"fp16", "bf16", "fp32"}
    scales = [r["scale"] for r in META["cases"]["fp16_z2_clip"]["trajectory"]]
    assert max(scales) > 256 and min(scales) < 256                   # grow and halve
    arr = arrays("fp16_z2_clip")
    bad = from_bits(arr["s3_g2"], torch.float16, (16, 33))
    assert not torch.isfinite(bad).all()


def _replays_cleanly(name) -> bool:
    case = META["cases"][name]
    arr = arrays(name)
    eng, params = _oracle_engine(case, arr)
    dtype = DTYPES[case["config"]["dtype"]]
    stage = case["config"]["zero_optimization"]["stage"]
    for step, rec in enumerate(case["trajectory"]):
        if stage >= 3:
            eng.gather_parameters()
        for p, g in zip(params, case_grads(case, arr, step, dtype)):
            p.grad = g
        eng.micro_steps += 1
        if eng.step() != rec["applied"] or eng.scaler.scale != rec["scale"]:
            return False
        for gi, g in enumerate(eng.groups):
            if not np.array_equal(g.data.numpy(), arr[f"s{step}_master{gi}"]):
                return False
            if not np.array_equal(eng.state[gi]["exp_avg_sq"].numpy(), arr[f"s{step}_v{gi}"]):
                return False
    return True


def _adam_no_decay(shard, grad, m, v, lr, betas, eps, wd, step_t):
    return _REAL_ADAM(shard, grad, m, v, lr, betas, eps, 0.0, step_t)


def _adam_no_bias_correction(shard, grad, m, v, lr, betas, eps, wd, step_t):
    if wd != 0.0:
        shard.add_(shard, alpha=-lr * wd)
    m.mul_(betas[0]).add_(grad, alpha=1.0 - betas[0])
    v.mul_(betas[1]).addcmul_(grad, grad, value=1.0 - betas[1])
    shard.addcdiv_(m, v.sqrt().add_(eps), value=-lr)


def _adam_swapped_betas(shard, grad, m, v, lr, betas, eps, wd, step_t):
    return _REAL_ADAM(shard, grad, m, v, lr, (betas[1], betas[0]), eps, wd, step_t)


def _adam_wrong_sign(shard, grad, m, v, lr, betas, eps, wd, step_t):
    return _REAL_ADAM(shard, grad, m, v, -lr, betas, eps, wd, step_t)


def _adam_fused_division(shard, grad, m, v, lr, betas, eps, wd, step_t):
    """Same maths, one rounding moved: (-lr) * (m_hat / den) instead of
    ((-lr) * m_hat) / den."""
    if wd != 0.0:
        shard.add_(shard, alpha=-lr * wd)
    m.mul_(betas[0]).add_(grad, alpha=1.0 - betas[0])
    v.mul_(betas[1]).addcmul_(grad, grad, value=1.0 - betas[1])
    denom = (v / (1.0 - betas[1] ** step_t)).sqrt().add_(eps)
    shard.add_((m / (1.0 - betas[0] ** step_t)) / denom, alpha=-lr)


_REAL_ADAM = ob.adam_update


@pytest.mark.parametrize("mutant", [_adam_no_decay, _adam_no_bias_correction, _adam_swapped_betas,
                                    _adam_wrong_sign, _adam_fused_division],
                         ids=lambda f: f.__name__)
def test_golden_vectors_catch_planted_adam_mistakes(monkeypatch, mutant):
    assert all(_replays_cleanly(n) for n in ("fp16_z2_clip", "fp32_z0_clip_adam"))
    monkeypatch.setattr(ob, "adam_update", mutant)
    assert not all(_replays_cleanly(n) for n in ("fp16_z2_clip", "fp32_z0_clip_adam"))


def test_golden_vectors_catch_planted_clip_and_scale_mistakes(monkeypatch):
    # clip on >= instead of > is invisible here; dropping the +1e-6 is not
    orig = ob.Engine.clip_gradients

    def no_eps(self, max_norm, clip_override=None):
        local = torch.zeros((), dtype=torch.float32)
        for g in self.groups:
            local += g.local_grad_sumsq()
        norm = float(local.sqrt().item())
        if max_norm is not None and norm > max_norm:
            for g in self.groups:
                g.scale_grads(max_norm / norm)
        return norm

    monkeypatch.setattr(ob.Engine, "clip_gradients", no_eps)
    assert not _replays_cleanly("fp16_z2_clip")
    monkeypatch.setattr(ob.Engine, "clip_gradients", orig)

    def update_no_reset(self, overflow):
        if not self.enabled:
            return
        if overflow:
            self.scale = max(self.scale / 2.0, self.min_scale)
            self.skipped_steps += 1
        else:
            self.good_steps += 1
            if self.good_steps >= self.scale_window and self.scale < self.max_scale:
                self.scale = min(self.scale * 2.0, self.max_scale)
                self.good_steps = 0

    monkeypatch.setattr(ob.LossScaler, "update", update_no_reset)
    assert not _replays_cleanly("fp16_z2_clip")


@pytest.mark.parametrize("name", ["fp16_z2_clip", "fp32_z0_clip_adam", "bf16_z1_noclip_2groups"])
def test_clip_override_with_the_own_decision_replays_the_reference(name):
    """The oracle's clip override (used by GPU tests to run the AdamW
    arithmetic on the GPU's own clip coefficient) reproduces minispeed's
    recorded trajectory when handed the decision the oracle itself makes."""
    case = META["cases"][name]
    arr = arrays(name)
    eng, params = _oracle_engine(case, arr)
    probe, probe_params = _oracle_engine(case, arr)
    dtype = DTYPES[case["config"]["dtype"]]
    stage = case["config"]["zero_optimization"]["stage"]
    clip = case["config"].get("gradient_clipping")
    for step, rec in enumerate(case["trajectory"]):
        grads = case_grads(case, arr, step, dtype)
        for ps, e in ((params, eng), (probe_params, probe)):
            if stage >= 3:
                e.gather_parameters()
            for p, g in zip(ps, grads):
                p.grad = None if g is None else g.clone()
            e.micro_steps += 1
        probe.step()                                   # the oracle's own decision
        norm = probe.grad_norm
        applied = bool(clip) and norm is not None and norm > clip
        override = (applied, clip / (norm + 1e-6) if applied else 1.0)
        assert eng.step(clip_override=override) == rec["applied"], step
        for gi, g in enumerate(eng.groups):
            np.testing.assert_array_equal(g.data.numpy(), arr[f"s{step}_master{gi}"])
            np.testing.assert_array_equal(eng.state[gi]["exp_avg"].numpy(), arr[f"s{step}_m{gi}"])
            np.testing.assert_array_equal(eng.state[gi]["exp_avg_sq"].numpy(), arr[f"s{step}_v{gi}"])


def test_mlp_traces_catch_a_planted_loss_scaling_mistake(monkeypatch):
    """The traces pin ``_scale_loss``: an oracle that forgets the division by
    gas, or scales by a different factor, no longer reproduces them."""
    def no_gas(self, loss):
        factor = self.scaler.loss_scale_factor
        return loss if factor == 1.0 else loss * factor

    for mutant in (no_gas,):
        monkeypatch.setattr(ob.Engine, "scale_loss", mutant)
        for name in ("mlp_fp32_trace", "mlp_fp16_trace"):
            with pytest.raises(AssertionError):
                test_oracle_matches_reference_mlp_trace(name)
