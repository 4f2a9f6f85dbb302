"""Write golden vectors of minispeed's boundary step by running minispeed.

    python tests/golden/make_golden.py [--reference /root/reference]

Runs only where minispeed's sources are (they never travel with this
repository; the fixtures do).  It imports
the reference package from ``--reference`` and drives its CPU engine
(``MINISPEED_DEVICE=cpu``) through seeded cases that exercise the hot path:
ragged parameter lists, fp16 / bf16 / fp32, ZeRO stages 0-3 at world size 1,
clipping on and off, dynamic and static loss scales, inf/nan injection,
parameters without a gradient, two groups with different hyper-parameters,
and the LR schedules.  Gradients are written straight into ``param.grad``
between boundaries (the engine's micro-step counter is advanced as
``backward`` would), so every input of every boundary is recorded exactly.

Three engine-level traces (an MLP trained through autograd: fp32 and bf16 at
gas 2, fp16 with a dynamic loss scale starting at 2^20 and window 2 at gas 3)
record losses, every boundary's outcome (applied or skipped, loss-scale
state, grad_norm, lr) and the final parameters; they pin the host-side loss
scaling of ``backward`` (loss * scale / gas), the accumulation of
micro-batch gradients in the parameter dtype and the boundary gating.  A third runs the tiny decoder LM of
``tests/tinylm.py`` (3.3M parameters, fp32, ZeRO 0, 20 steps) and records
its losses, gradient norms and per-tensor parameter sums (``cases.json`` key
``tinylm``): an end-to-end trace through autograd, compared on the GPU at a
tolerance that allows for CPU/GPU floating-point differences.

Three cases also write a checkpoint with minispeed's own
``engine.save_checkpoint`` part-way through (``CHECKPOINTS``: case -> number
of boundaries before the save) into ``ckpt/<case>/``; the trajectory after
the save pins a resume from minispeed's files.

Outputs, next to this script: ``<case>.npz`` (arrays, loaded with
``allow_pickle=False``; rewritten only when an array changed),
``ckpt/<case>/`` and ``cases.json`` (per-case configuration and scalar
trajectories).
"""

from __future__ import annotations

import argparse
import json
import os
import shutil
import sys

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))

SHAPES = [(7, 5), (3,), (16, 33), (1,), (129,)]


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw storage of a tensor as an integer array (fp16/bf16 -> int16)."""
    t = t.detach().contiguous().reshape(-1)
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().copy()
    return t.view(torch.int32).numpy().copy()


class Holder(nn.Module):
    def __init__(self, params):
        super().__init__()
        self.ps = nn.ParameterList([nn.Parameter(p.clone()) for p in params])


def make_params(seed: int, shapes):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(*s, generator=g) * 0.02 for s in shapes]


def base_cfg(dtype, stage, clip, lr=1e-3, wd=0.01, betas=(0.9, 0.999), eps=1e-8,
             opt_type="AdamW", scheduler="WarmupLR", sched_params=None, fp16=None, gas=1):
    cfg = {
        "train_micro_batch_size_per_gpu": 1,
        "gradient_accumulation_steps": gas,
        "gradient_clipping": clip,
        "dtype": dtype,
        "optimizer": {"type": opt_type, "params": {"lr": lr, "betas": list(betas), "eps": eps,
                                                   "weight_decay": wd}},
        "scheduler": {"type": scheduler, "params": dict(sched_params or {})},
        "zero_optimization": {"stage": stage},
        "steps_per_print": 1000,
    }
    if fp16 is not None:
        cfg["fp16"] = dict(fp16, enabled=True)
    return cfg


CASES = {
    "fp16_z2_clip": dict(
        cfg=base_cfg("fp16", 2, 1.0, scheduler="WarmupDecayLR",
                     sched_params={"warmup_min_lr": 0.0, "warmup_max_lr": 1e-3,
                                   "warmup_num_steps": 2, "total_num_steps": 10},
                     fp16={"loss_scale": 0, "initial_scale_power": 8, "loss_scale_window": 2}),
        groups=[list(range(5))], steps=8, std=0.1,
        inject={3: [("inf", 2, 5)], 5: [("nan", 0, 0)]}, none={6: [3]}),
    "bf16_z1_noclip_2groups": dict(
        cfg=base_cfg("bf16", 1, 0, scheduler="WarmupLR",
                     sched_params={"warmup_min_lr": 0.0, "warmup_num_steps": 3}),
        groups=[[0, 2], [1, 4, 3]],
        group_opts=[{}, {"lr": 5e-4, "weight_decay": 0.0, "betas": (0.8, 0.99)}],
        steps=6, std=1e-2, inject={}, none={}),
    "fp32_z0_clip_adam": dict(
        cfg=base_cfg("fp32", 0, 0.05, wd=0.1, eps=1e-6, opt_type="Adam"),
        groups=[list(range(5))], steps=5, std=1e-2, inject={}, none={2: [0, 4]}),
    "fp16_z3_overflow": dict(
        cfg=base_cfg("fp16", 3, 1.0,
                     fp16={"loss_scale": 0, "initial_scale_power": 4, "loss_scale_window": 3}),
        groups=[list(range(5))], steps=7, std=0.05,
        inject={2: [("-inf", 1, 2)], 3: [("nan", 4, 128)]}, none={}),
    "fp16_static_scale": dict(
        cfg=base_cfg("fp16", 0, 1.0,
                     fp16={"loss_scale": 1000.0, "initial_scale_power": 16, "loss_scale_window": 2}),
        groups=[list(range(5))], steps=5, std=0.1, inject={}, none={}),
}


CHECKPOINTS = {"fp16_z2_clip": 4, "bf16_z1_noclip_2groups": 3, "fp16_z3_overflow": 3}


def run_case(ms, name, spec, out_arrays, meta):
    torch.manual_seed(0)
    init = make_params(100, SHAPES)
    model = Holder(init)
    ps = list(model.ps)
    opts = spec.get("group_opts")
    if len(spec["groups"]) == 1 and not opts:
        model_parameters = [ps[i] for i in spec["groups"][0]]
    else:
        model_parameters = [dict({"params": [ps[i] for i in idx]}, **(opts[k] if opts else {}))
                            for k, idx in enumerate(spec["groups"])]
    engine = ms.initialize(model=model, model_parameters=model_parameters, config=spec["cfg"])
    stage = spec["cfg"]["zero_optimization"]["stage"]
    for i, t in enumerate(init):
        out_arrays[f"init_p{i}"] = t.numpy().copy()
    gen = torch.Generator().manual_seed(200)
    traj = []
    for step in range(spec["steps"]):
        if stage >= 3:
            engine.optimizer.gather_parameters()   # what engine.forward does
        scale = engine.loss_scaler.loss_scale_factor
        dtype = ps[0].dtype
        for i, p in enumerate(ps):
            g32 = torch.randn(SHAPES[i], generator=gen) * spec["std"] * scale
            if i in spec["none"].get(step, []):
                p.grad = None
                out_arrays[f"s{step}_g{i}_none"] = np.array([1], dtype=np.int8)
                continue
            g = g32.to(dtype)
            for kind, pi, idx in spec["inject"].get(step, []):
                if pi == i:
                    g.view(-1)[idx] = {"inf": float("inf"), "-inf": float("-inf"),
                                       "nan": float("nan")}[kind]
            p.grad = g
            out_arrays[f"s{step}_g{i}"] = bits(g)
        engine.micro_steps += 1                     # what engine.backward does
        applied = engine.step()
        rec = {
            "applied": bool(applied),
            "grad_norm": engine.grad_norm,
            "scale": engine.loss_scaler.scale,
            "good_steps": engine.loss_scaler.good_steps,
            "skipped_steps": engine.loss_scaler.skipped_steps,
            "global_steps": engine.global_steps,
            "lr": [float(g["lr"]) for g in engine.optimizer.param_groups],
            "adam_step": [int(st["step"]) for st in engine.optimizer.state],
        }
        traj.append(rec)
        if CHECKPOINTS.get(name) == step + 1:
            ckpt_root = os.path.join(HERE, "ckpt", name)
            shutil.rmtree(ckpt_root, ignore_errors=True)
            ckpt_dir = engine.save_checkpoint(ckpt_root)
            meta.setdefault("_checkpoints", {})[name] = {
                "after_steps": step + 1, "tag": os.path.basename(ckpt_dir)}
        for gi, fg in enumerate(engine.flat_groups):
            out_arrays[f"s{step}_master{gi}"] = fg.data.numpy().copy()
            st = engine.optimizer.state[gi]
            out_arrays[f"s{step}_m{gi}"] = st["exp_avg"].numpy().copy()
            out_arrays[f"s{step}_v{gi}"] = st["exp_avg_sq"].numpy().copy()
        for i, p in enumerate(ps):
            out_arrays[f"s{step}_model{i}"] = bits(p.data)
    ckpt = meta.pop("_checkpoints", {}).get(name)
    meta[name] = {"config": spec["cfg"], "groups": spec["groups"],
                  "group_opts": [{k: list(v) if isinstance(v, tuple) else v for k, v in o.items()}
                                 for o in (opts or [])],
                  "shapes": SHAPES, "steps": spec["steps"], "trajectory": traj}
    if ckpt:
        meta[name]["checkpoint"] = ckpt


class MLP(nn.Module):
    """The 8 -> 32 -> 32 -> 1 MLP of minispeed's tests/common.py:19-32."""

    def __init__(self):
        super().__init__()
        self.net = nn.Sequential(nn.Linear(8, 32), nn.Tanh(), nn.Linear(32, 32), nn.ReLU(),
                                 nn.LayerNorm(32), nn.Linear(32, 1))

    def forward(self, x):
        return self.net(x)


def run_mlp_trace(ms, name, dtype, out_arrays, meta, steps=4, gas=2, micro=4, fp16=None):
    torch.manual_seed(1234)
    model = MLP()
    for i, p in enumerate(model.parameters()):
        out_arrays[f"init_p{i}"] = p.detach().numpy().copy()
    g = torch.Generator().manual_seed(7)
    x = torch.randn(steps * gas * micro, 8, generator=g).view(steps, gas, micro, 8)
    y = torch.randn(steps * gas * micro, 1, generator=g).view(steps, gas, micro, 1)
    out_arrays["x"] = x.numpy().copy()
    out_arrays["y"] = y.numpy().copy()
    cfg = base_cfg(dtype, 0, 1.0, scheduler="WarmupDecayLR",
                   sched_params={"warmup_min_lr": 0.0, "warmup_max_lr": 1e-2,
                                 "warmup_num_steps": 1, "total_num_steps": 6},
                   lr=1e-2, gas=gas, fp16=fp16)
    cfg["train_micro_batch_size_per_gpu"] = micro
    engine = ms.initialize(model=model, model_parameters=list(model.parameters()), config=cfg)
    losses, boundaries = [], []
    for s in range(steps):
        for mi in range(gas):
            loss = F.mse_loss(engine(x[s, mi]).float(), y[s, mi].float())
            losses.append(float(loss.detach()))
            engine.backward(loss)
            applied = engine.step()
            if engine.is_gradient_accumulation_boundary:
                sc = engine.loss_scaler
                boundaries.append({"applied": bool(applied), "scale": sc.scale,
                                   "good_steps": sc.good_steps, "skipped_steps": sc.skipped_steps,
                                   "grad_norm": engine.grad_norm,
                                   "lr": [g["lr"] for g in engine.optimizer.param_groups],
                                   "global_steps": engine.global_steps})
    for i, p in enumerate(model.parameters()):
        out_arrays[f"final_p{i}"] = bits(p.data)
    out_arrays["final_master0"] = engine.flat_groups[0].data.numpy().copy()
    meta[name] = {"config": cfg, "steps": steps, "gas": gas, "micro": micro,
                  "losses": losses, "grad_norm": engine.grad_norm,
                  "global_steps": engine.global_steps, "boundaries": boundaries}


def run_tinylm_trace(ms, meta, steps=20):
    import copy

    if REPO not in sys.path:
        sys.path.insert(0, REPO)
    from tests import tinylm

    model = tinylm.build(0)
    engine = ms.initialize(model=model, model_parameters=list(model.parameters()),
                           config=copy.deepcopy(tinylm.CONFIG))
    data = tinylm.batches(steps, seed=1)
    losses, norms = [], []
    for s in range(steps):
        idx = data[s]
        loss = tinylm.loss_fn(engine(idx[:, :-1]), idx)
        losses.append(float(loss.detach()))
        engine.backward(loss)
        assert engine.step()
        norms.append(float(engine.grad_norm))
    sums = {name: [float(p.detach().double().sum()), float(p.detach().double().pow(2).sum())]
            for name, p in model.named_parameters()}
    meta["tinylm"] = {"config": tinylm.CONFIG, "steps": steps, "init_seed": 0, "data_seed": 1,
                      "losses": losses, "grad_norms": norms, "global_steps": engine.global_steps,
                      "param_sum_sumsq": sums}


def save_npz(name, arrays):
    """Write ``<name>.npz`` unless it already holds exactly these arrays
    (the zip container stamps times, so rewriting would churn the file)."""
    path = os.path.join(HERE, f"{name}.npz")
    if os.path.exists(path):
        with np.load(path, allow_pickle=False) as z:
            same = sorted(z.files) == sorted(arrays) and all(
                z[k].dtype == arrays[k].dtype and np.array_equal(z[k], arrays[k], equal_nan=True)
                for k in arrays)
        if same:
            return
    np.savez_compressed(path, **arrays)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args(argv)
    os.environ["MINISPEED_DEVICE"] = "cpu"
    os.environ["MINISPEED_BACKEND"] = "gloo"
    for key in ("RANK", "WORLD_SIZE", "LOCAL_RANK"):
        os.environ.pop(key, None)
    sys.path.insert(0, args.reference)
    import minispeed as ms  # the reference package

    torch.set_num_threads(1)
    meta = {"torch": torch.__version__, "cases": {}}
    for name, spec in CASES.items():
        arrays = {}
        run_case(ms, name, spec, arrays, meta["cases"])
        save_npz(name, arrays)
    for name, dtype in (("mlp_fp32_trace", "fp32"), ("mlp_bf16_trace", "bf16")):
        arrays = {}
        run_mlp_trace(ms, name, dtype, arrays, meta["cases"])
        save_npz(name, arrays)
    # fp16 with a dynamic scale and gas 3: the loss is multiplied by
    # scale / 3, a factor that rounds, and the first boundaries overflow
    arrays = {}
    run_mlp_trace(ms, "mlp_fp16_trace", "fp16", arrays, meta["cases"], steps=10, gas=3,
                  fp16={"loss_scale": 0, "initial_scale_power": 20, "loss_scale_window": 2})
    save_npz("mlp_fp16_trace", arrays)
    run_tinylm_trace(ms, meta)
    with open(os.path.join(HERE, "cases.json"), "w", encoding="utf-8") as fh:
        json.dump(meta, fh, indent=1, sort_keys=True)
    print("wrote", sorted(meta["cases"]))


if __name__ == "__main__":
    main()
