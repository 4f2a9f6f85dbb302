"""The reference's unfused step pieces, run on the HIP kernels.

minispeed's boundary (engine.py:268-322) is flatten_grads -> has_overflow ->
unscale_grads -> reduce_gradients -> clip_gradients -> optimizer.step ->
sync_parameters.  The engine here fuses them into K1-K3; the pieces are kept
as methods (flat.py:232-257, stage_1_and_2.py:86-128, stage_3.py:120-126)
for callers that drive them one by one.  Each piece is checked against
torch's CPU op on the same bits (``div_`` / ``mul_`` by a Python float:
IEEE division / one rounded multiply by the fp32-rounded scalar), the sum of
squares against float64, and the whole unfused sequence against the fused
``engine.step()`` of a twin engine.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch
from torch import nn

import minispeed_amd as ms
from minispeed_amd import precision
from tests.helpers import DEV, bits

pytestmark = pytest.mark.gpu


def _cfg(stage, dtype="fp16", clip=1.0):
    cfg = {"train_micro_batch_size_per_gpu": 1, "gradient_accumulation_steps": 1,
           "gradient_clipping": clip, "dtype": dtype,
           "optimizer": {"type": "AdamW", "params": {"lr": 1e-3, "betas": [0.9, 0.999],
                                                      "eps": 1e-8, "weight_decay": 0.01}},
           "zero_optimization": {"stage": stage}, "steps_per_print": 1000}
    if dtype == "fp16":
        cfg["fp16"] = {"enabled": True, "initial_scale_power": 12}
    return cfg


def _model():
    torch.manual_seed(3)
    return nn.Sequential(nn.Linear(67, 129), nn.GELU(), nn.Linear(129, 33), nn.LayerNorm(33))


def _set_grads(module, seed, scale):
    gen = torch.Generator().manual_seed(seed)
    for p in module.parameters():
        p.grad = (torch.randn(p.shape, generator=gen) * 1e-2 * scale).to(p.dtype).to(DEV)


@pytest.mark.parametrize("stage", [1, 2])
def test_unscale_scale_and_sumsq_match_torch(stage):
    module = _model().to(DEV)
    engine = ms.initialize(model=module, model_parameters=list(module.parameters()), config=_cfg(stage))
    g = engine.flat_groups[0]
    _set_grads(module, 0, 4096.0)
    g.flatten_grads()
    engine.optimizer.reduce_gradients()
    for scale in (4096.0, 1000.0, 3.0):
        before = g.grad.cpu()
        g.unscale_grads(scale)
        np.testing.assert_array_equal(bits(g.grad), bits(before.div_(scale)))
    target = g.grad_shard if stage >= 2 else g.grad
    for factor in (0.37, 1.0 / 3.0, 2.0):
        before = target.cpu()
        g.scale_grads(factor)
        np.testing.assert_array_equal(bits(target), bits(before.mul_(factor)))
    s = g.local_grad_sumsq()
    assert s.dtype == torch.float32 and s.dim() == 0 and s.device.type == "cuda"
    exact = float((g.grad_for_shard().double() ** 2).sum())
    assert abs(float(s) - exact) <= 1e-6 * exact


def test_scale_by_zero_and_empty_buffers():
    module = _model().to(DEV)
    engine = ms.initialize(model=module, model_parameters=list(module.parameters()), config=_cfg(1))
    g = engine.flat_groups[0]
    _set_grads(module, 1, 1.0)
    g.flatten_grads()
    g.scale_grads(0.0)
    assert int(g.grad.count_nonzero()) == 0
    assert float(g.local_grad_sumsq()) == 0.0
    with pytest.raises(RuntimeError):
        g.unscale_grads(-2.0)        # a loss scale must be positive
    from minispeed_amd.boundary import scale_in_place, sumsq_device
    empty = torch.empty(0, device=DEV)
    scale_in_place(empty, ms._native.SCALE_MULTIPLY, 3.0)
    assert float(sumsq_device(empty)) == 0.0


@pytest.mark.parametrize("stage", [0, 1, 2, 3])
@pytest.mark.parametrize("clip", [1e-3, 100.0])
def test_unfused_sequence_equals_the_fused_boundary(stage, clip):
    """flatten -> overflow -> unscale -> reduce -> clip -> step -> sync on
    one engine, engine.step() on its twin: same norm, masters, moments and
    model parameters, bit for bit."""
    base = _model()
    mods = [copy.deepcopy(base).to(DEV) for _ in range(2)]
    engines = [ms.initialize(model=m, model_parameters=list(m.parameters()), config=_cfg(stage, clip=clip))
               for m in mods]
    unfused, fused = engines
    opt = unfused.optimizer
    scale = unfused.loss_scaler.scale
    for step in range(2):
        if stage >= 3:
            opt.gather_parameters()
            fused.optimizer.gather_parameters()
        for m in mods:
            _set_grads(m, 10 + step, scale)

        for g in unfused.flat_groups:
            g.flatten_grads()
        assert not precision.has_overflow(*[g.grad for g in unfused.flat_groups])
        for g in unfused.flat_groups:
            g.unscale_grads(scale)
        opt.reduce_gradients()
        norm = opt.clip_gradients(clip)
        opt.step()
        opt.sync_parameters()

        fused.micro_steps += 1
        assert fused.step() is True
        # both sum the same fp32 values over the same K1 block ranges; the
        # norms agree exactly, and so does everything after them
        assert norm == fused.grad_norm
        if stage >= 3:
            opt.gather_parameters()
            fused.optimizer.gather_parameters()
        for a, b in zip(unfused.flat_groups, fused.flat_groups):
            np.testing.assert_array_equal(bits(a.data), bits(b.data))
        for sa, sb in zip(opt.state, fused.optimizer.state):
            assert sa["step"] == sb["step"] == step + 1
            np.testing.assert_array_equal(bits(sa["exp_avg"]), bits(sb["exp_avg"]))
            np.testing.assert_array_equal(bits(sa["exp_avg_sq"]), bits(sb["exp_avg_sq"]))
        for pa, pb in zip(mods[0].parameters(), mods[1].parameters()):
            np.testing.assert_array_equal(bits(pa), bits(pb))
        for g in unfused.flat_groups:
            g.zero_grad()
        if stage >= 3:
            for g in unfused.flat_groups:
                assert g.grad is None
