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
from tests.helpers import relative_within

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


def _close(got, want, scale, where):
    """Per element |got - want| <= 1e-5 * max(|want|, scale), ``scale`` the
    element's largest magnitude along minispeed's recorded run (an element
    passing near zero is held to its own size, not the buffer's)."""
    ok, worst = relative_within(got, want, scale)
    assert ok, (where, worst)


def _run_scale(arr, key, upto, *extra):
    """Each element's largest magnitude in minispeed's record of ``key``
    (``s{step}_<key>``) over steps 0 .. upto, and in ``extra``."""
    out = np.zeros_like(np.asarray(arr[f"s0_{key}"], np.float32))
    for s in range(upto + 1):
        np.maximum(out, np.abs(arr[f"s{s}_{key}"]), out=out)
    for x in extra:
        np.maximum(out, np.abs(np.asarray(x, np.float32)), out=out)
    return out


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
            st = engine.optimizer.state[gi]
            for key, got in ((f"master{gi}", g.data), (f"m{gi}", st["exp_avg"]),
                             (f"v{gi}", st["exp_avg_sq"])):
                got = got.cpu().numpy()
                _close(got, arr[f"s{step}_{key}"], _run_scale(arr, key, step, got), (step, key))
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
    for gi, (a, b) in enumerate(zip(mine["fp32_groups"], theirs["fp32_groups"])):
        _close(a.numpy(), b.numpy(), _run_scale(arr, f"master{gi}", k - 1, a), "fp32_groups")
    for gi, (a, b) in enumerate(zip(mine["optimizer"]["shard_state"],
                                    theirs["optimizer"]["shard_state"])):
        assert a["step"] == b["step"]
        _close(a["exp_avg"].numpy(), b["exp_avg"].numpy(),
               _run_scale(arr, f"m{gi}", k - 1, a["exp_avg"]), "exp_avg")
        _close(a["exp_avg_sq"].numpy(), b["exp_avg_sq"].numpy(),
               _run_scale(arr, f"v{gi}", k - 1, a["exp_avg_sq"]), "exp_avg_sq")
    mod_mine = _load(os.path.join(out, ckpt.MODEL_STATES))
    mod_theirs = _load(os.path.join(ref_root, tag, ckpt.MODEL_STATES))
    assert mod_mine["tag"] == mod_theirs["tag"] == tag
    assert set(mod_mine["module"]) == set(mod_theirs["module"])
    # the saved parameters are the cast of the saved masters, bit for bit
    # (the masters are held to minispeed's above)
    name_of = {id(p): name for name, p in engine.module.named_parameters()}
    for g, masters in zip(engine.flat_groups, mine["fp32_groups"]):
        lo = g.master_range[0]
        for (off, p), n in zip(g._offsets, g._numels):
            saved = mod_mine["module"][name_of[id(p)]]
            want = masters[off - lo:off - lo + n].to(saved.dtype).reshape(saved.shape)
            np.testing.assert_array_equal(bits_of(saved), bits_of(want), err_msg=name_of[id(p)])
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
