"""Checkpoints in minispeed's on-disk format (minispeed/checkpoint.py).

    <save_dir>/latest                                      newest tag (text)
    <save_dir>/<tag>/mp_rank_00_model_states.pt            {"module", "tag"}
    <save_dir>/<tag>/zero_pp_rank<r>_mp_rank_00_optim_states.pt
        {"optimizer": {"param_groups", "shard_state": [{"step", "exp_avg",
         "exp_avg_sq"}]}, "fp32_groups": [masters per group],
         "lr_scheduler", "loss_scaler", "global_steps", "micro_steps",
         "grad_norm", "rank", "world_size"}

The same file names and keys as checkpoint.py:21-125, so a run can resume
from a checkpoint minispeed wrote and minispeed can resume from one written
here.  Tensors are stored on the CPU; files are read with
``torch.load(..., weights_only=True)``.
"""

from __future__ import annotations

import os
from typing import Optional, Tuple

import torch

from . import comm

MODEL_STATES = "mp_rank_00_model_states.pt"
LATEST = "latest"


def optim_states_name(rank: int) -> str:
    return f"zero_pp_rank{rank}_mp_rank_00_optim_states.pt"


def _cpu(obj):
    if isinstance(obj, torch.Tensor):
        return obj.detach().cpu().clone()
    if isinstance(obj, dict):
        return {k: _cpu(v) for k, v in obj.items()}
    if isinstance(obj, list):
        return [_cpu(v) for v in obj]
    if isinstance(obj, tuple):
        return tuple(_cpu(v) for v in obj)
    return obj


def read_latest(save_dir: str) -> str:
    with open(os.path.join(save_dir, LATEST), "r", encoding="utf-8") as fh:
        return fh.read().strip()


@torch.no_grad()
def save_checkpoint(engine, save_dir: str, tag: Optional[str] = None) -> str:
    """Write the model state (rank 0), ``latest`` and this rank's optimizer
    shard; ZeRO-3 parameters are gathered for the model state and freed
    again afterwards (checkpoint.py:35-71)."""
    tag = tag or f"global_step{engine.global_steps}"
    ckpt_dir = os.path.join(save_dir, tag)
    os.makedirs(ckpt_dir, exist_ok=True)
    was_gathered = engine.optimizer.params_gathered
    engine.optimizer.gather_parameters()
    if engine.rank == 0:
        torch.save({"module": _cpu(engine.module.state_dict()), "tag": tag},
                   os.path.join(ckpt_dir, MODEL_STATES))
        with open(os.path.join(save_dir, LATEST), "w", encoding="utf-8") as fh:
            fh.write(tag)
    state = {
        "optimizer": _cpu(engine.optimizer.state_dict()),
        "fp32_groups": [g.data.detach().cpu().clone() for g in engine.flat_groups],
        "lr_scheduler": engine.lr_scheduler.state_dict(),
        "loss_scaler": engine.loss_scaler.state_dict(),
        "global_steps": engine.global_steps,
        "micro_steps": engine.micro_steps,
        "grad_norm": engine.grad_norm,
        "rank": engine.rank,
        "world_size": engine.world_size,
    }
    torch.save(state, os.path.join(ckpt_dir, optim_states_name(engine.rank)))
    comm.barrier()
    if not was_gathered:
        engine.optimizer.free_parameters()
    return ckpt_dir


@torch.no_grad()
def load_checkpoint(engine, load_dir: str, tag: Optional[str] = None) -> Tuple[str, dict]:
    """Restore model, masters, optimizer shard, scheduler, scaler and
    counters (checkpoint.py:74-125).  Masters are restored from the saved
    fp32 buffers and cast into the model parameters on the GPU."""
    tag = tag or read_latest(load_dir)
    ckpt_dir = os.path.join(load_dir, tag)
    was_gathered = engine.optimizer.params_gathered
    engine.optimizer.gather_parameters()

    model_state = torch.load(os.path.join(ckpt_dir, MODEL_STATES), map_location="cpu",
                             weights_only=True)
    engine.module.load_state_dict(model_state["module"])

    optim_path = os.path.join(ckpt_dir, optim_states_name(engine.rank))
    if not os.path.exists(optim_path):
        raise FileNotFoundError(f"Missing optimizer shard for rank {engine.rank}: {optim_path}")
    state = torch.load(optim_path, map_location="cpu", weights_only=True)
    saved_world = int(state.get("world_size", engine.world_size))
    if saved_world != engine.world_size:
        raise RuntimeError(
            f"Checkpoint was saved with world_size={saved_world} but current "
            f"world_size={engine.world_size}; ZeRO shards do not transfer."
        )
    if len(state["fp32_groups"]) != len(engine.flat_groups):
        raise RuntimeError(
            f"checkpoint has {len(state['fp32_groups'])} parameter groups, "
            f"the engine {len(engine.flat_groups)}")
    for g, buf in zip(engine.flat_groups, state["fp32_groups"]):
        if buf.numel() != g.data.numel():
            raise RuntimeError(f"master buffer of {buf.numel()} elements, expected {g.data.numel()}")
        g.data.copy_(buf)
        g.copy_flat_to_model()
    if engine.config.zero_stage >= 3:
        engine.optimizer.free_parameters()
        if was_gathered:
            engine.optimizer.gather_parameters()
    engine.optimizer.load_state_dict(state["optimizer"])
    engine.lr_scheduler.load_state_dict(state["lr_scheduler"])
    engine.loss_scaler.load_state_dict(state["loss_scaler"])
    engine.global_steps = int(state.get("global_steps", 0))
    engine.micro_steps = int(state.get("micro_steps", 0))
    engine.grad_norm = state.get("grad_norm")
    comm.barrier()
    return tag, state
