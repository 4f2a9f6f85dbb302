"""Torch-CPU restatement of minispeed's boundary step (the oracle).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Every device computation is the same ATen op, in the same order, with the
same scalar arguments as the reference, so on one torch CPU build the
results are minispeed's bits.  Each function names the reference lines it
restates.  World size 1 only, plus the layout of "rank r of W" for shard
arithmetic.
"""

from __future__ import annotations

from typing import List, Optional, Sequence

import torch
from torch import nn


# ----------------------------------------------------------------- layout
def round_up(x: int, m: int) -> int:                       # flat.py:16-17
    return ((x + m - 1) // m) * m


class Group:
    """FlatParamGroup (flat.py:20-260) on CPU, holding real nn.Parameters."""

    def __init__(self, params: Sequence[nn.Parameter], rank: int = 0, world_size: int = 1,
                 zero_stage: int = 0):
        self.params = list(params)
        self.zero_stage = zero_stage
        self.numel = sum(p.numel() for p in self.params)                 # flat.py:50
        self.numel_padded = round_up(self.numel, world_size)             # flat.py:51
        self.shard_size = self.numel_padded // world_size                # flat.py:52
        if zero_stage >= 1:                                               # flat.py:54-59
            self.shard_start = rank * self.shard_size
            self.shard_end = self.shard_start + self.shard_size
        else:
            self.shard_start, self.shard_end = 0, self.numel_padded
        self.data = torch.zeros(self.numel_padded, dtype=torch.float32)  # flat.py:61
        self.grad = None if zero_stage >= 3 else torch.zeros(self.numel_padded)   # flat.py:64-68
        self.grad_shard = torch.zeros(self.shard_size) if zero_stage >= 2 else None  # flat.py:69-73
        self.offsets, self.numels, self.shapes = [], [], []               # flat.py:78-86
        off = 0
        for p in self.params:
            self.offsets.append(off)
            self.numels.append(p.numel())
            self.shapes.append(tuple(p.shape))
            off += p.numel()
        self.partitioned = False

    def master_range(self):                                               # flat.py:91-100
        return (self.shard_start, self.shard_end) if self.partitioned else (0, self.numel_padded)

    def pdata_range(self, off: int, n: int, p: nn.Parameter):             # flat.py:103-113
        if p.data.numel() == n:
            return off, off + n
        s = max(off, self.shard_start)
        return s, s + p.data.numel()

    @torch.no_grad()
    def copy_model_to_flat(self):                                         # flat.py:115-131
        ms, me = self.master_range()
        for off, n, p in zip(self.offsets, self.numels, self.params):
            ps, pe = self.pdata_range(off, n, p)
            lo, hi = max(ps, ms), min(pe, me)
            if lo < hi:
                self.data[lo - ms:hi - ms].copy_(p.data.reshape(-1)[lo - ps:hi - ps])

    @torch.no_grad()
    def copy_flat_to_model(self, full: Optional[torch.Tensor] = None):    # flat.py:133-154
        buf, base = (full, 0) if full is not None else (self.data, self.master_range()[0])
        end = base + buf.numel()
        for off, n, p in zip(self.offsets, self.numels, self.params):
            ps, pe = self.pdata_range(off, n, p)
            lo, hi = max(ps, base), min(pe, end)
            if lo < hi:
                p.data.view(-1)[lo - ps:hi - ps].copy_(buf[lo - base:hi - base])

    @torch.no_grad()
    def partition_params(self):                                           # flat.py:157-172
        if self.partitioned:
            return
        self.data = self.data[self.shard_start:self.shard_end].clone()
        self.partitioned = True
        self.dematerialize_params()
        self.copy_flat_to_model()

    @torch.no_grad()
    def materialize_params(self):                                         # flat.py:174-181
        if self.partitioned:
            for p, shape in zip(self.params, self.shapes):
                p.data = torch.empty(shape, dtype=p.data.dtype)

    @torch.no_grad()
    def dematerialize_params(self):                                       # flat.py:183-193
        if not self.partitioned:
            return
        for off, n, p in zip(self.offsets, self.numels, self.params):
            lo, hi = max(off, self.shard_start), min(off + n, self.shard_end)
            p.data = torch.empty(max(0, hi - lo), dtype=p.data.dtype)

    @torch.no_grad()
    def flatten_grads(self):                                              # flat.py:196-213
        if self.grad is None:
            self.grad = torch.zeros(self.numel_padded, dtype=torch.float32)
        else:
            self.grad.zero_()
        for off, n, p in zip(self.offsets, self.numels, self.params):
            if p.grad is None:
                continue
            self.grad[off:off + n].copy_(p.grad.data.reshape(-1))
            p.grad = None

    @torch.no_grad()
    def zero_grad(self):                                                  # flat.py:215-223
        if self.grad is not None:
            if self.zero_stage >= 3:
                self.grad = None
            else:
                self.grad.zero_()
        if self.grad_shard is not None:
            self.grad_shard.zero_()

    def grad_for_shard(self):                                             # flat.py:225-229
        if self.grad_shard is not None:
            return self.grad_shard
        return self.grad[self.shard_start:self.shard_end]

    def local_grad_sumsq(self):                                           # flat.py:232-234
        return self.grad_for_shard().pow(2).sum()

    @property
    def shard(self):                                                      # flat.py:236-241
        return self.data if self.partitioned else self.data[self.shard_start:self.shard_end]

    @torch.no_grad()
    def unscale_grads(self, scale: float):                                # flat.py:243-247
        if scale == 1.0 or self.grad is None:
            return
        self.grad.div_(scale)

    @torch.no_grad()
    def scale_grads(self, factor: float):                                 # flat.py:249-257
        if factor == 1.0:
            return
        if self.grad_shard is not None:
            self.grad_shard.mul_(factor)
        elif self.grad is not None:
            self.grad.mul_(factor)


# -------------------------------------------------------------- precision
class LossScaler:
    """DynamicLossScaler (precision.py:10-76)."""

    def __init__(self, enabled=True, init_scale=0.0, scale_window=1000, min_scale=1.0,
                 max_scale=2.0 ** 24):
        self.enabled, self.min_scale, self.max_scale = enabled, min_scale, max_scale
        self.scale_window = max(1, scale_window)
        if not enabled:
            self.scale = 1.0
        elif init_scale and init_scale > 0:
            self.scale = float(init_scale)
        else:
            self.scale = 1.0
        self.good_steps = 0
        self.skipped_steps = 0

    def set_scale_from_power(self, power):                                # precision.py:42-44
        if self.enabled:
            self.scale = float(2.0 ** int(power))

    @property
    def loss_scale_factor(self):                                          # precision.py:46-48
        return self.scale if self.enabled else 1.0

    def update(self, overflow: bool):                                     # precision.py:50-62
        if not self.enabled:
            return
        if overflow:
            self.scale = max(self.scale / 2.0, self.min_scale)
            self.good_steps = 0
            self.skipped_steps += 1
        else:
            self.good_steps += 1
            if self.good_steps >= self.scale_window and self.scale < self.max_scale:
                self.scale = min(self.scale * 2.0, self.max_scale)
                self.good_steps = 0


def has_overflow(*bufs) -> bool:                                          # precision.py:79-87
    for b in bufs:
        if b is None or b.numel() == 0:
            continue
        if not torch.isfinite(b).all():
            return True
    return False


# -------------------------------------------------------------- scheduler
class Schedule:
    """WarmupLR / WarmupDecayLR (scheduler.py:12-99); kind in {"WarmupLR",
    "WarmupDecayLR"}."""

    def __init__(self, param_groups, kind="WarmupLR", warmup_min_lr=0.0, warmup_max_lr=1e-3,
                 warmup_num_steps=0, total_num_steps=None):
        self.param_groups = param_groups
        self.kind = kind
        self.min_lr, self.max_lr = float(warmup_min_lr), float(warmup_max_lr)
        self.warm = max(0, int(warmup_num_steps))
        self.total = None if total_num_steps is None else int(total_num_steps)
        self.last_epoch = -1                                              # scheduler.py:31

    def _warmup(self, e):                                                 # scheduler.py:37-44
        if self.warm <= 0:
            return self.max_lr
        if e < self.warm:
            return self.min_lr + (self.max_lr - self.min_lr) * (e / self.warm)
        return self.max_lr

    def get_lr(self):
        e = self.last_epoch
        if self.kind == "WarmupLR":                                       # scheduler.py:76-77
            return self._warmup(e)
        if e < self.warm:                                                 # scheduler.py:84-95
            return self._warmup(e)
        if self.total is None:
            return self.max_lr
        if e >= self.total:
            return self.min_lr
        frac = (self.total - e) / max(1, self.total - self.warm)
        return self.min_lr + (self.max_lr - self.min_lr) * frac

    def step(self):                                                       # scheduler.py:50-54
        self.last_epoch += 1
        lr = self.get_lr()
        for g in self.param_groups:
            g["lr"] = lr

    def get_last_lr(self):
        return float(self.param_groups[0]["lr"])


# ----------------------------------------------------------------- AdamW
@torch.no_grad()
def adam_update(shard, grad, m, v, lr, betas, eps, wd, step_t):         # adam.py:77-100
    """One FlatAdam update of one group (``step_t`` already incremented)."""
    beta1, beta2 = betas
    if wd != 0.0:
        shard.add_(shard, alpha=-lr * wd)
    m.mul_(beta1).add_(grad, alpha=1.0 - beta1)
    v.mul_(beta2).addcmul_(grad, grad, value=1.0 - beta2)
    bias_c1 = 1.0 - beta1 ** step_t
    bias_c2 = 1.0 - beta2 ** step_t
    denom = (v / bias_c2).sqrt().add_(eps)
    shard.addcdiv_(m / bias_c1, denom, value=-lr)


# ------------------------------------------------------------------ engine
class Engine:
    """The boundary-step part of DeepSpeedEngine (engine.py:84-322) plus the
    ZeRO optimizer it drives (stage_1_and_2.py, stage_3.py), world size 1.

    ``groups`` are lists of nn.Parameters (fp32 at construction, as the
    reference expects); ``opts`` are per-group dicts with lr / betas / eps /
    weight_decay.
    """

    def __init__(self, groups: List[List[nn.Parameter]], opts: List[dict], *, dtype="fp32",
                 zero_stage=0, clip: Optional[float] = None, gas=1, loss_scale=0.0,
                 initial_scale_power=16, loss_scale_window=1000, scheduler="WarmupLR",
                 scheduler_params: Optional[dict] = None, rank=0, world_size=1):
        self.zero_stage = zero_stage
        self.clip = clip
        self.gas = gas
        self.groups = [Group(ps, rank, world_size, zero_stage) for ps in groups]
        for g in self.groups:
            g.copy_model_to_flat()                                        # engine.py:114-115
        self.dtype = {"fp32": None, "fp16": torch.float16, "bf16": torch.bfloat16}[dtype]
        if self.dtype is not None:                                        # engine.py:118-124
            for g in self.groups:
                for p in g.params:
                    p.data = p.data.to(self.dtype)
        if zero_stage >= 3:                                               # engine.py:127-129
            for g in self.groups:
                g.partition_params()
        self.param_groups = []
        self.state = []
        for g, o in zip(self.groups, opts):                               # adam.py:50-65
            d = dict(o)
            d.setdefault("lr", 1e-3)
            d.setdefault("betas", (0.9, 0.999))
            d.setdefault("eps", 1e-8)
            d.setdefault("weight_decay", 0.0)
            self.param_groups.append(d)
            n = g.shard_end - g.shard_start
            self.state.append({"step": 0, "exp_avg": torch.zeros(n), "exp_avg_sq": torch.zeros(n)})
        sp = dict(scheduler_params or {})
        sp.setdefault("warmup_max_lr", float(self.param_groups[0]["lr"]))
        self.scheduler = Schedule(self.param_groups, scheduler,
                                  sp.get("warmup_min_lr", 0.0), sp["warmup_max_lr"],
                                  sp.get("warmup_num_steps", 0), sp.get("total_num_steps"))
        enabled = dtype == "fp16"                                         # engine.py:141-148
        self.scaler = LossScaler(enabled, loss_scale, loss_scale_window)
        if enabled and loss_scale == 0:
            self.scaler.set_scale_from_power(initial_scale_power)
        self.gathered = False
        self.global_steps = 0
        self.skipped_steps = 0
        self.micro_steps = 0
        self.grad_norm = None

    # -------------------------------------------------------- stage 3
    def gather_parameters(self):                                          # stage_3.py:67-86
        if self.zero_stage < 3 or self.gathered:
            return
        for g in self.groups:
            g.materialize_params()
            full = torch.empty(g.numel_padded, dtype=torch.float32)
            full.copy_(g.shard)                                           # comm.py:133-134
            g.copy_flat_to_model(full)
        self.gathered = True

    def free_parameters(self):                                            # stage_3.py:88-100
        if self.zero_stage < 3 or not self.gathered:
            return
        for g in self.groups:
            g.dematerialize_params()
            g.copy_flat_to_model()
        self.gathered = False

    def params_gathered(self):
        return self.zero_stage < 3 or self.gathered

    # ------------------------------------------------------- backward
    def scale_loss(self, loss):                                           # engine.py:227-233
        factor = self.scaler.loss_scale_factor
        if self.gas > 1:
            factor /= self.gas
        return loss if factor == 1.0 else loss * factor

    def backward(self, loss):                                             # engine.py:235-251
        self.scale_loss(loss).backward()
        self.micro_steps += 1

    # ----------------------------------------------------------- step
    def zero_grad(self):
        for g in self.groups:
            g.zero_grad()

    def reduce_gradients(self):                                           # stage_1_and_2.py:86-102
        for g in self.groups:
            if self.zero_stage >= 2:
                g.grad_shard.copy_(g.grad)                                # comm.py:124-125
        if self.zero_stage >= 3:                                          # stage_3.py:120-126
            for g in self.groups:
                g.grad = None

    def clip_gradients(self, max_norm, clip_override=None):               # stage_1_and_2.py:105-128
        """``clip_override`` = (applied, coefficient as a double) replaces
        the clip decision and coefficient derived from this norm, so that a
        test can run the AdamW arithmetic on exactly the gradients another
        implementation clipped (the norm itself is still this one)."""
        local = torch.zeros((), dtype=torch.float32)
        for g in self.groups:
            local += g.local_grad_sumsq()
        norm = float(local.sqrt().item())
        self.grad_norm_raw = local
        if clip_override is not None:
            applied, coef = clip_override
            if applied:
                for g in self.groups:
                    g.scale_grads(float(coef))
            return norm
        if max_norm is not None and norm > max_norm:
            coef = max_norm / (norm + 1e-6)
            for g in self.groups:
                g.scale_grads(coef)
        return norm

    def sync_parameters(self):                                            # stage_1_and_2.py:79-83
        if self.zero_stage >= 3:
            self.free_parameters()                                        # stage_3.py:102-110
        else:
            for g in self.groups:
                g.copy_flat_to_model()

    @torch.no_grad()
    def take_step(self, flat_grads=None, clip_override=None) -> bool:     # engine.py:268-322
        """``flat_grads`` (one fp32 flat tensor per group, numel_padded)
        stands in for the flatten of ``param.grad``: the boundary of the
        opt-in contiguous-gradient mode, which minispeed does not have; every
        later step is the reference's.  ``clip_override``: see
        :meth:`clip_gradients`."""
        if flat_grads is None:
            for g in self.groups:
                g.flatten_grads()
        else:
            for g, f in zip(self.groups, flat_grads):
                g.grad = f.to(torch.float32).clone()
                for p in g.params:
                    p.grad = None
        overflow = any(has_overflow(g.grad) for g in self.groups)
        if overflow:
            self.scaler.update(overflow=True)
            self.skipped_steps += 1
            self.zero_grad()
            self.free_parameters()
            return False
        scale = self.scaler.loss_scale_factor
        if scale != 1.0:
            for g in self.groups:
                g.unscale_grads(scale)
        self.reduce_gradients()
        self.grad_norm = self.clip_gradients(self.clip, clip_override)
        for group, g, st in zip(self.param_groups, self.groups, self.state):   # adam.py:59-93
            st["step"] += 1
            lr = float(group["lr"])
            b1, b2 = group["betas"]
            adam_update(g.shard, g.grad_for_shard(), st["exp_avg"], st["exp_avg_sq"], lr,
                        (b1, b2), float(group["eps"]), float(group.get("weight_decay", 0.0)),
                        st["step"])
        self.sync_parameters()
        self.scaler.update(overflow=False)
        self.scheduler.step()
        self.zero_grad()
        self.global_steps += 1
        return True

    def load_state(self, masters, exp_avgs, exp_avg_sqs, steps, scaler_state, lr_epoch,
                   lrs) -> None:
        """Start from a given state (fp32 tensors per group, Adam step
        counters, (scale, good_steps, skipped_steps), scheduler epoch, current
        lrs); the model parameters are refreshed from the masters."""
        for g, d, m, v, st, k, lr in zip(self.groups, masters, exp_avgs, exp_avg_sqs, self.state,
                                         steps, lrs):
            g.data.copy_(d)
            st["exp_avg"].copy_(m)
            st["exp_avg_sq"].copy_(v)
            st["step"] = int(k)
        for pg, lr in zip(self.param_groups, lrs):
            pg["lr"] = lr
        self.scaler.scale, self.scaler.good_steps, self.scaler.skipped_steps = scaler_state
        self.scheduler.last_epoch = lr_epoch
        for g in self.groups:
            if not g.partitioned:
                g.copy_flat_to_model()

    def step(self, flat_grads=None, clip_override=None) -> bool:          # engine.py:254-266
        if not (self.micro_steps > 0 and self.micro_steps % self.gas == 0):
            return False
        if getattr(self, "_consumed", -1) == self.micro_steps:
            return False
        self._consumed = self.micro_steps
        return self.take_step(flat_grads, clip_override)


def accumulate_fp32(acc: Optional[torch.Tensor], grad: torch.Tensor) -> torch.Tensor:
    """One micro-batch of the opt-in contiguous-gradient mode: the gradient
    widened to fp32 and added to the running fp32 sum (one rounding)."""
    g = grad.detach().reshape(-1).to(torch.float32)
    return g.clone() if acc is None else acc + g
