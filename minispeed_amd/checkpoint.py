"""Checkpoints in minispeed's on-disk format (minispeed/checkpoint.py).

    <save_dir>/latest                                      newest tag (text)
    <save_dir>/<tag>/mp_rank_00_model_states.pt            {"module", "tag"}
    <save_dir>/<tag>/zero_pp_rank<r>_mp_rank_00_optim_states.pt
        {"optimizer": {"param_groups", "shard_state": [{"step", "exp_avg",
         "exp_avg_sq"}]}, "fp32_groups": [masters per group],
         "lr_scheduler", "loss_scaler", "global_steps", "micro_steps",
         "grad_norm", "rank", "world_size"}

File names, keys and the two load errors are minispeed's
(checkpoint.py:21-125), so either implementation resumes from the other's
files.  Everything is written as CPU tensors (the flat buffers live in HBM
here) and read with ``torch.load(..., weights_only=True)``.

The model state needs full-shaped parameters; at ZeRO-3 the parameters are
placeholders between steps, so both directions run inside
:func:`_full_parameters`, which gathers them and afterwards returns them to
the state they were in.
"""

from __future__ import annotations

import os
from contextlib import contextmanager
from dataclasses import dataclass
from typing import Iterator, Optional, Tuple

import torch

from . import comm

MODEL_STATES = "mp_rank_00_model_states.pt"
LATEST = "latest"

# keys of the per-rank file that are plain engine counters: (key, attribute, cast)
_COUNTERS = (("global_steps", "global_steps", int), ("micro_steps", "micro_steps", int),
             ("grad_norm", "grad_norm", None))


def optim_states_name(rank: int) -> str:
    return f"zero_pp_rank{rank}_mp_rank_00_optim_states.pt"


def read_latest(save_dir: str) -> str:
    with open(os.path.join(save_dir, LATEST), "r", encoding="utf-8") as fh:
        return fh.read().strip()


@dataclass(frozen=True)
class _Where:
    root: str
    tag: str

    @property
    def folder(self) -> str:
        return os.path.join(self.root, self.tag)

    @property
    def model_file(self) -> str:
        return os.path.join(self.folder, MODEL_STATES)

    def shard_file(self, rank: int) -> str:
        return os.path.join(self.folder, optim_states_name(rank))


def _to_host(obj):
    """Deep copy with every tensor on the CPU (device buffers can be views
    of larger allocations; a copy stores only their own elements)."""
    if isinstance(obj, torch.Tensor):
        return obj.detach().to("cpu", copy=True)
    if isinstance(obj, (list, tuple)):
        return type(obj)(_to_host(v) for v in obj)
    if isinstance(obj, dict):
        return {k: _to_host(v) for k, v in obj.items()}
    return obj


@contextmanager
def _full_parameters(engine, refresh: bool = False) -> Iterator[None]:
    """Full-shaped parameters inside the block; afterwards the ZeRO-3
    placeholders come back if that is how the block found them.  With
    ``refresh`` (after new masters were loaded) a ZeRO-3 engine is freed and
    re-gathered, so the parameters are recast from the masters."""
    opt = engine.optimizer
    gathered_before = opt.params_gathered
    opt.gather_parameters()
    ok = False
    try:
        yield
        ok = True
    finally:
        # also when the block raised (a missing shard, a size mismatch, a
        # disk error): the ZeRO-3 placeholders come back, and after a failed
        # load the parameters (which the module's load_state_dict may already
        # have overwritten) are recast from the masters, which a failed load
        # leaves untouched
        if refresh and engine.config.zero_stage >= 3:
            opt.free_parameters()
            if gathered_before:
                opt.gather_parameters()
        else:
            if refresh and not ok:
                for g in engine.flat_groups:
                    g.copy_flat_to_model()
            if not gathered_before:
                opt.free_parameters()


def _shard_payload(engine) -> dict:
    payload = {
        "optimizer": _to_host(engine.optimizer.state_dict()),
        "fp32_groups": [_to_host(g.data) for g in engine.flat_groups],
        "lr_scheduler": engine.lr_scheduler.state_dict(),
        "loss_scaler": engine.loss_scaler.state_dict(),
    }
    payload.update({key: getattr(engine, attr) for key, attr, _ in _COUNTERS})
    payload["rank"], payload["world_size"] = engine.rank, engine.world_size
    return payload


def _restore_masters(engine, saved) -> None:
    groups = engine.flat_groups
    if len(saved) != len(groups):
        raise RuntimeError(f"checkpoint has {len(saved)} parameter groups, the engine {len(groups)}")
    for g, buf in zip(groups, saved):      # every group checked before any is written
        if buf.numel() != g.data.numel():
            raise RuntimeError(f"master buffer of {buf.numel()} elements, expected {g.data.numel()}")
    for g, buf in zip(groups, saved):
        g.data.copy_(buf)
        g.copy_flat_to_model()


@torch.no_grad()
def save_checkpoint(engine, save_dir: str, tag: Optional[str] = None) -> str:
    """Rank 0 writes the model state and ``latest``; every rank writes its
    optimizer shard (checkpoint.py:35-71).  Returns the checkpoint folder."""
    where = _Where(save_dir, tag or f"global_step{engine.global_steps}")
    os.makedirs(where.folder, exist_ok=True)
    with _full_parameters(engine):
        if engine.rank == 0:
            torch.save({"module": _to_host(engine.module.state_dict()), "tag": where.tag},
                       where.model_file)
            with open(os.path.join(save_dir, LATEST), "w", encoding="utf-8") as fh:
                fh.write(where.tag)
        torch.save(_shard_payload(engine), where.shard_file(engine.rank))
        comm.barrier()
    return where.folder


@torch.no_grad()
def load_checkpoint(engine, load_dir: str, tag: Optional[str] = None) -> Tuple[str, dict]:
    """Model state, masters (cast into the parameters on the GPU), optimizer
    shard, scheduler, scaler and counters (checkpoint.py:74-125).  Returns
    ``(tag, the per-rank file's contents)``."""
    where = _Where(load_dir, tag or read_latest(load_dir))
    shard_file = where.shard_file(engine.rank)
    with _full_parameters(engine, refresh=True):
        model = torch.load(where.model_file, map_location="cpu", weights_only=True)
        engine.module.load_state_dict(model["module"])
        if not os.path.exists(shard_file):
            raise FileNotFoundError(f"Missing optimizer shard for rank {engine.rank}: {shard_file}")
        state = torch.load(shard_file, map_location="cpu", weights_only=True)
        saved_world = int(state.get("world_size", engine.world_size))
        if saved_world != engine.world_size:
            raise RuntimeError(
                f"Checkpoint was saved with world_size={saved_world} but current "
                f"world_size={engine.world_size}; ZeRO shards do not transfer.")
        _restore_masters(engine, state["fp32_groups"])
    engine.optimizer.load_state_dict(state["optimizer"])
    engine.lr_scheduler.load_state_dict(state["lr_scheduler"])
    engine.loss_scaler.load_state_dict(state["loss_scaler"])
    for key, attr, cast in _COUNTERS:
        value = state.get(key, 0 if cast else None)
        setattr(engine, attr, cast(value) if cast else value)
    comm.barrier()
    return where.tag, state
