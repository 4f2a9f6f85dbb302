"""ZeRO-3 gather/free as views of one model-dtype buffer (world size 1).

The freed placeholders and the gathered parameters are views into
``FlatParamGroup.model_shard``: gather and free allocate nothing, and the
gathered parameters always equal the reference's cast-on-gather of the
current masters (stage_3.py:67-86), bit for bit, whatever happened since the
last cast: a boundary with or without a gather, a skipped boundary, a
standalone optimizer step, in-place writes to the masters or the
parameters, a checkpoint load, a write through a freed placeholder's
``.data``.  By default every gather casts, as the reference's does; with
``hip_boundary.stage3_gather_reuse`` the gather runs no cast when the buffer
already holds the cast of the masters by the version counters, and a write
through a placeholder's ``.data`` (which they do not see) survives it.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F
from torch import nn

import minispeed_amd as ms

pytestmark = pytest.mark.gpu
DEV = "cuda"


class MLP(nn.Module):
    def __init__(self):
        super().__init__()
        self.net = nn.Sequential(nn.Linear(8, 32), nn.Tanh(), nn.Linear(32, 32), nn.ReLU(),
                                 nn.LayerNorm(32), nn.Linear(32, 1))

    def forward(self, x):
        return self.net(x)


def _engine(dtype="fp16", reuse=False):
    torch.manual_seed(0)
    model = MLP().to(DEV)
    cfg = {"train_micro_batch_size_per_gpu": 4, "gradient_accumulation_steps": 1,
           "gradient_clipping": 1.0, "dtype": dtype,
           "optimizer": {"type": "AdamW", "params": {"lr": 1e-2, "weight_decay": 0.01}},
           "zero_optimization": {"stage": 3}, "hip_boundary": {"stage3_gather_reuse": reuse}}
    if dtype == "fp16":
        cfg["fp16"] = {"enabled": True, "loss_scale": 0, "initial_scale_power": 8}
    engine = ms.initialize(model=model, model_parameters=list(model.parameters()), config=cfg)
    return engine, model


def _batch(seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(4, 8, generator=g).to(DEV), torch.randn(4, 1, generator=g).to(DEV)


def _train_step(engine, seed):
    x, y = _batch(seed)
    engine.backward(F.mse_loss(engine(x).float(), y))
    return engine.step()


class CastCounter:
    """Counts casts into the model copy issued through copy_flat_to_model."""

    def __init__(self, group):
        self.n = 0
        orig = group.copy_flat_to_model

        def counted(*a, **k):
            self.n += 1
            return orig(*a, **k)

        group.copy_flat_to_model = counted


def _assert_gathered_is_cast_of_masters(engine, model):
    g = engine.flat_groups[0]
    assert engine.optimizer.params_gathered
    base = g.model_shard.data_ptr()
    esz = g.model_shard.element_size()
    for (off, p), n in zip(g._offsets, g._numels):
        assert p.data_ptr() == base + off * esz            # a view, not a copy
        want = g.data[off:off + n].to(p.dtype).view(p.shape)
        assert torch.equal(p.data.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("reuse", [False, True])
def test_gather_and_free_are_views_that_allocate_nothing(reuse):
    engine, model = _engine(reuse=reuse)
    assert engine.optimizer.gather_reuse is reuse
    g = engine.flat_groups[0]
    counter = CastCounter(g)
    assert _train_step(engine, 1) is True
    assert not engine.optimizer.params_gathered
    ms_, me = g.shard_start, g.shard_end
    for (off, p), n in zip(g._offsets, g._numels):
        assert p.dim() == 1 and p.numel() == n
        assert p.data_ptr() == g.model_shard.data_ptr() + off * g.model_shard.element_size()
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    n0 = counter.n
    engine.optimizer.gather_parameters()
    assert counter.n == n0 + (0 if reuse else 1)            # reuse: fresh, no cast
    assert torch.cuda.memory_allocated() == before
    _assert_gathered_is_cast_of_masters(engine, model)
    engine.optimizer.free_parameters()
    assert torch.cuda.memory_allocated() == before


@pytest.mark.parametrize("event", ["boundary_without_gather", "standalone_step", "masters_inplace",
                                   "param_inplace", "skipped_boundary", "load_state_dict"])
def test_gather_recasts_whenever_the_copy_may_be_stale(event):
    """With gather_reuse: the cast is skipped only while the version
    counters show the buffer holds the cast of the current masters."""
    engine, model = _engine(reuse=True)
    g = engine.flat_groups[0]
    for s in range(2):
        assert _train_step(engine, 10 + s) is True
    counter = CastCounter(g)
    if event == "boundary_without_gather":
        # gradients on the freed placeholders, then a boundary: the masters
        # move but the placeholders keep their values, as in the reference
        for p in model.parameters():
            p.grad = torch.full_like(p, 0.5)
        engine.micro_steps += 1
        old = g.model_shard.clone()
        assert engine.step() is True
        assert torch.equal(g.model_shard, old)
    elif event == "standalone_step":
        g.grad_shard.fill_(0.25)
        engine.optimizer.step()
    elif event == "masters_inplace":
        g.data.mul_(1.5)
    elif event == "param_inplace":
        with torch.no_grad():
            next(model.parameters()).add_(1.0)               # a freed placeholder
    elif event == "skipped_boundary":
        x, y = _batch(20)
        engine.backward(F.mse_loss(engine(x).float(), y))
        next(model.parameters()).grad.view(-1)[0] = float("inf")
        assert engine.step() is False
    elif event == "load_state_dict":
        sd = {k: v.clone() * 0.5 for k, v in engine.state_dict().items()}
        engine.optimizer.free_parameters()
        engine.load_state_dict(sd)
        engine.optimizer.free_parameters()
    n0 = counter.n
    engine.optimizer.gather_parameters()
    if event in ("skipped_boundary", "load_state_dict"):
        assert counter.n == n0            # already recast by the free that followed
    else:
        assert counter.n == n0 + 1
    _assert_gathered_is_cast_of_masters(engine, model)
    # and training goes on from there
    assert _train_step(engine, 30) is True
    engine.optimizer.gather_parameters()
    _assert_gathered_is_cast_of_masters(engine, model)


@pytest.mark.parametrize("reuse", [False, True])
def test_write_through_a_freed_placeholder_data(reuse):
    """A write through a freed placeholder's ``.data`` (torch's version
    counters do not see it).  minispeed's gather builds new parameters from
    the cast of the masters, so the write is gone (stage_3.py:67-86): the
    default gather does the same.  With gather_reuse the write survives the
    gather, the documented price of skipping the cast."""
    engine, model = _engine(reuse=reuse)
    g = engine.flat_groups[0]
    for s in range(2):
        assert _train_step(engine, 40 + s) is True
    assert not engine.optimizer.params_gathered
    first = next(model.parameters())
    first.data.fill_(3.0)                            # no version bump
    engine.optimizer.gather_parameters()
    if reuse:
        assert bool((first.data == 3.0).all())
    else:
        _assert_gathered_is_cast_of_masters(engine, model)
        assert not bool((first.data == 3.0).any())
    engine.optimizer.free_parameters()               # refreshed from the masters either way
    engine.optimizer.gather_parameters()
    _assert_gathered_is_cast_of_masters(engine, model)
    assert _train_step(engine, 50) is True


def test_views_train_like_stage0_bitwise():
    """The zero-copy gather changes no numerics: stage 3 equals stage 0."""
    out = []
    for stage in (0, 3):
        torch.manual_seed(0)
        model = MLP().to(DEV)
        cfg = {"train_micro_batch_size_per_gpu": 4, "gradient_accumulation_steps": 2,
               "gradient_clipping": 1.0, "dtype": "bf16",
               "optimizer": {"type": "AdamW", "params": {"lr": 1e-2, "weight_decay": 0.01}},
               "zero_optimization": {"stage": stage}}
        engine = ms.initialize(model=model, model_parameters=list(model.parameters()), config=cfg)
        losses = []
        for s in range(6):
            x, y = _batch(100 + s)
            loss = F.mse_loss(engine(x).float(), y)
            losses.append(float(loss.detach()))
            engine.backward(loss)
            engine.step()
        engine.optimizer.gather_parameters()
        out.append((losses, [p.detach().clone() for p in model.parameters()],
                    engine.flat_groups[0].data.clone()))
    assert out[0][0] == out[1][0]
    assert torch.equal(out[0][2], out[1][2])
    for a, b in zip(out[0][1], out[1][1]):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
