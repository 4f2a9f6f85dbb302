"""Checkpoints on the GPU: minispeed's on-disk layout both ways.

* A checkpoint written by minispeed's own ``save_checkpoint`` part-way
  through a recorded case (tests/golden/ckpt/) is loaded into this engine,
  which then continues the case: every later boundary must match the
  recorded trajectory (step applied or skipped, loss-scale state, lr, Adam
  step counters and global steps exactly; grad_norm within 1e-5 relative;
  masters within 1e-5 relative).
* A checkpoint written here for the same case has minispeed's file names and
  the same key tree, Python types, tensor dtypes and shapes as the one
  minispeed wrote, and the same scalar state; its tensors are within the
  trajectory tolerance of minispeed's (1e-5 relative), so minispeed's
  ``load_checkpoint`` (checkpoint.py:74-125) reads it as its own.
* Save, train on, load, train again replays bit for bit, at ZeRO stages 0
  and 3 (minispeed tests/test_engine.py:129-156, tests/test_zero3.py:150-181,
  which ask for 1e-5).
"""

from __future__ import annotations

import copy
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch import nn

import minispeed_amd as ms
from minispeed_amd import checkpoint as ckpt
from tests.golden_cases import (CHECKPOINT_CASES, DTYPES, META, Holder, arrays, bits_of,
                                case_grads, checkpoint_root)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _engine(case, arr):
    params = [nn.Parameter(torch.from_numpy(arr[f"init_p{i}"].copy()).to(DEV))
              for i in range(len(case["shapes"]))]
    module = Holder(params)
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
    return engine, list(module.ps)


def _boundary(engine, params, case, arr, step):
    dtype = DTYPES[case["config"]["dtype"]]
    if case["config"]["zero_optimization"]["stage"] >= 3:
        engine.optimizer.gather_parameters()
    for p, g in zip(params, case_grads(case, arr, step, dtype)):
        p.grad = None if g is None else g.to(DEV)
    engine.micro_steps += 1
    return engine.step()


def _assert_state(engine, rec, where):
    s = engine.loss_scaler
    assert (s.scale, s.good_steps, s.skipped_steps) == (
        rec["scale"], rec["good_steps"], rec["skipped_steps"]), where
    assert [g["lr"] for g in engine.optimizer.param_groups] == rec["lr"], where
    assert [st["step"] for st in engine.optimizer.state] == rec["adam_step"], where
    assert engine.global_steps == rec["global_steps"], where
    if rec["grad_norm"] is None:
        assert engine.grad_norm is None, where
    else:
        assert abs(engine.grad_norm - rec["grad_norm"]) <= 1e-5 * rec["grad_norm"], where


def _close(got, want, where):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * float(np.abs(want).max() or 1.0),
                               err_msg=str(where))


@pytest.mark.parametrize("name", CHECKPOINT_CASES)
def test_resumes_from_a_checkpoint_minispeed_wrote(name):
    case = META["cases"][name]
    arr = arrays(name)
    k = case["checkpoint"]["after_steps"]
    stage = case["config"]["zero_optimization"]["stage"]
    engine, params = _engine(case, arr)

    tag, state = engine.load_checkpoint(checkpoint_root(name))
    assert tag == case["checkpoint"]["tag"]
    rec = case["trajectory"][k - 1]
    _assert_state(engine, rec, "after load")
    assert engine.micro_steps == k
    for gi, g in enumerate(engine.flat_groups):
        # the masters minispeed saved are the ones it recorded after boundary k
        np.testing.assert_array_equal(g.data.cpu().numpy(), arr[f"s{k - 1}_master{gi}"])
        st = engine.optimizer.state[gi]
        np.testing.assert_array_equal(st["exp_avg"].cpu().numpy(), arr[f"s{k - 1}_m{gi}"])
        np.testing.assert_array_equal(st["exp_avg_sq"].cpu().numpy(), arr[f"s{k - 1}_v{gi}"])
    if stage >= 3:
        assert not engine.optimizer.params_gathered
        engine.optimizer.gather_parameters()
    for i, p in enumerate(params):
        np.testing.assert_array_equal(bits_of(p.data), arr[f"s{k - 1}_model{i}"])

    for step in range(k, case["steps"]):
        rec = case["trajectory"][step]
        assert _boundary(engine, params, case, arr, step) == rec["applied"], step
        _assert_state(engine, rec, step)
        for gi, g in enumerate(engine.flat_groups):
            _close(g.data.cpu().numpy(), arr[f"s{step}_master{gi}"], (step, gi))
            st = engine.optimizer.state[gi]
            _close(st["exp_avg"].cpu().numpy(), arr[f"s{step}_m{gi}"], (step, gi, "m"))
            _close(st["exp_avg_sq"].cpu().numpy(), arr[f"s{step}_v{gi}"], (step, gi, "v"))
        if stage >= 3:
            assert not engine.optimizer.params_gathered


def _tree(obj):
    """Key tree of a checkpoint with leaves reduced to type / dtype / shape."""
    if isinstance(obj, dict):
        return {k: _tree(v) for k, v in obj.items()}
    if isinstance(obj, (list, tuple)):
        return (type(obj).__name__, [_tree(v) for v in obj])
    if isinstance(obj, torch.Tensor):
        return ("tensor", str(obj.dtype), tuple(obj.shape))
    return type(obj).__name__


def _load(path):
    return torch.load(path, map_location="cpu", weights_only=True)


@pytest.mark.parametrize("name", CHECKPOINT_CASES)
def test_saved_checkpoint_has_minispeed_layout(name, tmp_path):
    case = META["cases"][name]
    arr = arrays(name)
    k = case["checkpoint"]["after_steps"]
    tag = case["checkpoint"]["tag"]
    engine, params = _engine(case, arr)
    for step in range(k):
        _boundary(engine, params, case, arr, step)
    out = engine.save_checkpoint(str(tmp_path))
    assert out == os.path.join(str(tmp_path), tag)
    ref_root = checkpoint_root(name)
    assert sorted(os.listdir(tmp_path)) == sorted(os.listdir(ref_root))
    assert ckpt.read_latest(str(tmp_path)) == ckpt.read_latest(ref_root) == tag
    assert sorted(os.listdir(out)) == sorted(os.listdir(os.path.join(ref_root, tag)))

    for fname in os.listdir(out):
        mine, theirs = _load(os.path.join(out, fname)), _load(os.path.join(ref_root, tag, fname))
        assert _tree(mine) == _tree(theirs), fname
    mine = _load(os.path.join(out, ckpt.optim_states_name(0)))
    theirs = _load(os.path.join(ref_root, tag, ckpt.optim_states_name(0)))
    for key in ("lr_scheduler", "loss_scaler", "global_steps", "micro_steps", "rank",
                "world_size"):
        assert mine[key] == theirs[key], key
    assert mine["optimizer"]["param_groups"] == theirs["optimizer"]["param_groups"]
    assert abs(mine["grad_norm"] - theirs["grad_norm"]) <= 1e-5 * theirs["grad_norm"]
    for a, b in zip(mine["fp32_groups"], theirs["fp32_groups"]):
        _close(a.numpy(), b.numpy(), "fp32_groups")
    for a, b in zip(mine["optimizer"]["shard_state"], theirs["optimizer"]["shard_state"]):
        assert a["step"] == b["step"]
        _close(a["exp_avg"].numpy(), b["exp_avg"].numpy(), "exp_avg")
        _close(a["exp_avg_sq"].numpy(), b["exp_avg_sq"].numpy(), "exp_avg_sq")
    mod_mine = _load(os.path.join(out, ckpt.MODEL_STATES))
    mod_theirs = _load(os.path.join(ref_root, tag, ckpt.MODEL_STATES))
    assert mod_mine["tag"] == mod_theirs["tag"] == tag
    for key, v in mod_theirs["module"].items():
        _close(mod_mine["module"][key].float().numpy(), v.float().numpy(), key)
    if case["config"]["zero_optimization"]["stage"] >= 3:
        assert not engine.optimizer.params_gathered   # save freed what it gathered


class MLP(nn.Module):
    def __init__(self):
        super().__init__()
        self.net = nn.Sequential(nn.Linear(8, 32), nn.Tanh(), nn.Linear(32, 32), nn.ReLU(),
                                 nn.LayerNorm(32), nn.Linear(32, 1))

    def forward(self, x):
        return self.net(x)


def _train(engine, x, y, steps, gas):
    losses = []
    for s in range(steps):
        for m in range(gas):
            loss = F.mse_loss(engine(x[s, m]).float(), y[s, m].float())
            losses.append(float(loss.detach()))
            engine.backward(loss)
            engine.step()
    return losses


@pytest.mark.parametrize("dtype,stage", [("fp32", 0), ("fp16", 0), ("bf16", 2), ("fp16", 3)])
def test_checkpoint_roundtrip_replays_bitwise(dtype, stage, tmp_path):
    gas, micro = 2, 4
    cfg = {"train_micro_batch_size_per_gpu": micro, "gradient_accumulation_steps": gas,
           "gradient_clipping": 1.0, "dtype": dtype,
           "optimizer": {"type": "AdamW", "params": {"lr": 1e-2, "betas": [0.9, 0.999],
                                                      "eps": 1e-8, "weight_decay": 0.01}},
           "scheduler": {"type": "WarmupDecayLR",
                         "params": {"warmup_min_lr": 0.0, "warmup_max_lr": 1e-2,
                                    "warmup_num_steps": 4, "total_num_steps": 40}},
           "zero_optimization": {"stage": stage}}
    if dtype == "fp16":
        cfg["fp16"] = {"enabled": True, "loss_scale": 0, "initial_scale_power": 6,
                       "loss_scale_window": 2}
    g = torch.Generator().manual_seed(7)
    x = torch.randn(4, gas, micro, 8, generator=g).to(DEV)
    y = torch.randn(4, gas, micro, 1, generator=g).to(DEV)
    torch.manual_seed(1234)
    model = MLP().to(DEV)
    engine = ms.initialize(model=model, model_parameters=list(model.parameters()), config=cfg)
    _train(engine, x, y, 2, gas)

    engine.save_checkpoint(str(tmp_path), tag="mid")
    if stage >= 3:
        assert not engine.optimizer.params_gathered
    expected_losses = _train(engine, x[2:], y[2:], 2, gas)
    expected_steps = engine.global_steps
    expected_scale = engine.get_loss_scale()
    expected_masters = [fg.data.clone() for fg in engine.flat_groups]
    if stage >= 3:
        engine.optimizer.gather_parameters()
    expected_params = {k: v.clone() for k, v in model.state_dict().items()}

    engine.load_checkpoint(str(tmp_path), tag="mid")
    assert engine.global_steps == expected_steps - 2
    replay_losses = _train(engine, x[2:], y[2:], 2, gas)
    assert replay_losses == expected_losses
    assert engine.global_steps == expected_steps and engine.get_loss_scale() == expected_scale
    for a, b in zip(engine.flat_groups, expected_masters):
        assert torch.equal(a.data, b)
    if stage >= 3:
        engine.optimizer.gather_parameters()
    for key, v in model.state_dict().items():
        assert torch.equal(v.view(torch.uint8), expected_params[key].view(torch.uint8)), key
