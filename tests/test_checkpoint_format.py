"""Checkpoint host logic on the CPU, against the checkpoints minispeed wrote
(tests/golden/ckpt/, by minispeed's checkpoint.py:35-71)."""

from __future__ import annotations

import os
import shutil
from types import SimpleNamespace

import pytest
import torch
from torch import nn

from minispeed_amd import checkpoint as ckpt
from tests.golden_cases import CHECKPOINT_CASES, META, Holder, checkpoint_root

OPTIM_KEYS = {"optimizer", "fp32_groups", "lr_scheduler", "loss_scaler", "global_steps",
              "micro_steps", "grad_norm", "rank", "world_size"}


def test_there_are_checkpoint_fixtures():
    assert {"fp16_z2_clip", "bf16_z1_noclip_2groups", "fp16_z3_overflow"} <= set(CHECKPOINT_CASES)


@pytest.mark.parametrize("name", CHECKPOINT_CASES)
def test_minispeed_checkpoints_use_the_names_and_keys_the_loader_reads(name):
    root = checkpoint_root(name)
    tag = ckpt.read_latest(root)
    assert tag == META["cases"][name]["checkpoint"]["tag"]
    files = sorted(os.listdir(os.path.join(root, tag)))
    assert files == sorted([ckpt.MODEL_STATES, ckpt.optim_states_name(0)])
    model = torch.load(os.path.join(root, tag, ckpt.MODEL_STATES), weights_only=True)
    assert set(model) == {"module", "tag"} and model["tag"] == tag
    state = torch.load(os.path.join(root, tag, ckpt.optim_states_name(0)), weights_only=True)
    assert set(state) == OPTIM_KEYS
    assert set(state["optimizer"]) == {"param_groups", "shard_state"}
    ngroups = len(META["cases"][name]["groups"])
    assert len(state["fp32_groups"]) == len(state["optimizer"]["shard_state"]) == ngroups
    for st, buf in zip(state["optimizer"]["shard_state"], state["fp32_groups"]):
        assert set(st) == {"step", "exp_avg", "exp_avg_sq"}
        assert buf.dtype == st["exp_avg"].dtype == torch.float32
        assert buf.shape == st["exp_avg"].shape == st["exp_avg_sq"].shape   # one rank


def _fake_engine(world_size=1, rank=0, ngroups=1, numel=696):
    params = [nn.Parameter(torch.zeros(s, dtype=torch.float16))
              for s in [(7, 5), (3,), (16, 33), (1,), (129,)]]
    opt = SimpleNamespace(params_gathered=True, gather_parameters=lambda: None,
                          free_parameters=lambda: None)
    groups = [SimpleNamespace(data=torch.zeros(numel), copy_flat_to_model=lambda: None)
              for _ in range(ngroups)]
    return SimpleNamespace(rank=rank, world_size=world_size, module=Holder(params),
                           optimizer=opt, flat_groups=groups,
                           config=SimpleNamespace(zero_stage=2))


class _TrackingOptimizer:
    """Stands in for a ZeRO-3 optimizer: records gathers, frees and the
    parameters' state, so a failed load can be checked for what it leaves."""

    def __init__(self, gathered):
        self.params_gathered = gathered
        self.calls = []

    def gather_parameters(self):
        self.calls.append("gather")
        self.params_gathered = True

    def free_parameters(self):
        self.calls.append("free")
        self.params_gathered = False


@pytest.mark.parametrize("stage", [2, 3])
@pytest.mark.parametrize("gathered", [False, True])
def test_failed_load_restores_the_parameters(stage, gathered):
    """A load that raises half-way (here: the rank's optimizer shard is
    missing, after the module's weights were loaded) leaves the ZeRO-3
    gather state as it found it and the parameters recast from the
    untouched masters."""
    eng = _fake_engine(rank=1)
    eng.config.zero_stage = stage
    eng.optimizer = _TrackingOptimizer(gathered)
    casts = []
    for g in eng.flat_groups:
        g.copy_flat_to_model = lambda g=g: casts.append(g)
    with pytest.raises(FileNotFoundError, match="rank 1"):
        ckpt.load_checkpoint(eng, checkpoint_root("fp16_z2_clip"))
    assert eng.optimizer.params_gathered is gathered
    if stage >= 3:
        assert "free" in eng.optimizer.calls          # placeholders refreshed from the masters
    else:
        assert casts == eng.flat_groups


def test_load_refuses_another_world_size():
    with pytest.raises(RuntimeError, match="world_size=1"):
        ckpt.load_checkpoint(_fake_engine(world_size=2), checkpoint_root("fp16_z2_clip"))


def test_load_names_the_missing_rank_shard(tmp_path):
    with pytest.raises(FileNotFoundError, match="rank 1"):
        ckpt.load_checkpoint(_fake_engine(rank=1), checkpoint_root("fp16_z2_clip"))


def test_load_refuses_a_different_group_layout():
    with pytest.raises(RuntimeError, match="parameter groups"):
        ckpt.load_checkpoint(_fake_engine(ngroups=2), checkpoint_root("fp16_z2_clip"))
    with pytest.raises(RuntimeError, match="elements"):
        ckpt.load_checkpoint(_fake_engine(numel=700), checkpoint_root("fp16_z2_clip"))


def test_explicit_tag_overrides_latest(tmp_path):
    src = checkpoint_root("fp16_z2_clip")
    dst = tmp_path / "run"
    shutil.copytree(src, dst)
    (dst / ckpt.LATEST).write_text("no-such-tag")
    tag = ckpt.read_latest(src)
    with pytest.raises(FileNotFoundError):
        ckpt.load_checkpoint(_fake_engine(), str(dst))
    with pytest.raises(RuntimeError, match="world_size=1"):
        ckpt.load_checkpoint(_fake_engine(world_size=3), str(dst), tag=tag)
