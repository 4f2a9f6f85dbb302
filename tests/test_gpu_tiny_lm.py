"""The tiny decoder LM workload end to end on the GPU.

The 4-layer GPT-style decoder of ``tests/tinylm.py`` (3,323,392 parameters in
52 tensors), fp32, ZeRO 0, AdamW lr 1e-3 betas (0.9,0.999) eps 1e-8 wd 0.01,
clip 1.0, 20 boundaries of one micro-batch of 8 x 128 tokens.

* Every boundary is checked against the oracle started from the GPU's own
  state with the gradients autograd produced on the GPU (copied before
  ``engine.step`` releases them) and the GPU's clip coefficient: norm
  within 1e-5, moments bit-exact, masters within 2 fp32 ulp per step.
* The whole run is compared with minispeed's own run of the same model,
  initialisation and token batches on the CPU (``cases.json`` key
  ``tinylm``, written by tests/golden/make_golden.py): losses within 2e-5
  relative, gradient norms within 1e-4 relative, per-tensor parameter sums
  of squares within 1e-4 relative and sums within 2e-4 of their L2 scale.
  These tolerances cover the different reduction orders of the CPU and GPU
  forward/backward kernels, which is the only difference between the runs
  (measured: 1.5e-7, 6.5e-7, 3.0e-6 and 1.7e-5; the margin allows for other
  GEMM algorithm choices on another box, and stays far below what a wrong
  boundary step does to a 20-step run).
"""

from __future__ import annotations

import copy
import math

import numpy as np
import pytest
import torch
from torch import nn

import minispeed_amd as ms
from minispeed_amd.workloads import numel, shapes_of
from oracle import boundary as ob
from tests import tinylm
from tests.golden_cases import META
from tests.helpers import clip_override, master_step_within_ulps, step_hyper

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_tiny_lm_trains_through_the_engine_and_matches_the_oracle_and_minispeed():
    trace = META["tinylm"]
    model = tinylm.build(trace["init_seed"]).to(DEV)
    shapes = [tuple(p.shape) for p in model.parameters()]
    assert shapes == shapes_of("tiny-lm-3.3m") and numel(shapes) == 3_323_392
    engine = ms.initialize(model=model, model_parameters=list(model.parameters()),
                           config=copy.deepcopy(tinylm.CONFIG))
    params = list(model.parameters())
    opt = tinylm.CONFIG["optimizer"]["params"]
    ref_params = [nn.Parameter(p.detach().cpu().clone()) for p in params]
    ref = ob.Engine([ref_params], [{"lr": opt["lr"], "betas": tuple(opt["betas"]), "eps": opt["eps"],
                                    "weight_decay": opt["weight_decay"]}], dtype="fp32",
                    zero_stage=0, clip=1.0, scheduler_params={"warmup_max_lr": opt["lr"]})
    data = tinylm.batches(trace["steps"], seed=trace["data_seed"]).to(DEV)
    g = engine.flat_groups[0]
    losses, norms = [], []
    for step in range(trace["steps"]):
        idx = data[step]
        loss = tinylm.loss_fn(engine(idx[:, :-1]), idx)
        losses.append(float(loss.detach()))
        engine.backward(loss)
        grads = [p.grad.detach().cpu().clone() for p in params]
        before = g.data.detach().cpu()
        st = engine.optimizer.state[0]
        ref.load_state([before], [st["exp_avg"].cpu()], [st["exp_avg_sq"].cpu()], [st["step"]],
                       (1.0, 0, 0), engine.lr_scheduler.last_epoch,
                       [pg["lr"] for pg in engine.optimizer.param_groups])
        for rp, gr in zip(ref_params, grads):
            rp.grad = gr
        ref.micro_steps += 1
        hp = step_hyper(engine)
        assert engine.step() is True and ref.step(clip_override=clip_override(engine)) is True
        norms.append(engine.grad_norm)
        assert abs(engine.grad_norm - ref.grad_norm) <= 1e-5 * ref.grad_norm
        ok, worst, nsq = master_step_within_ulps(before.numpy(), g.data.cpu().numpy(),
                                                 ref.groups[0].data.numpy(), st["exp_avg"].cpu().numpy(),
                                                 st["exp_avg_sq"].cpu().numpy(), **hp)
        assert ok, (step, worst, nsq)
        np.testing.assert_array_equal(st["exp_avg"].cpu().numpy(), ref.state[0]["exp_avg"].numpy())
        np.testing.assert_array_equal(st["exp_avg_sq"].cpu().numpy(), ref.state[0]["exp_avg_sq"].numpy())
        # fp32 model: the parameters are the masters
        for (off, p), n in zip(g._offsets, g._numels):
            assert torch.equal(p.detach().reshape(-1), g.data[off:off + n])
    assert engine.global_steps == trace["global_steps"] == trace["steps"]

    # against minispeed's own CPU run
    np.testing.assert_allclose(losses, trace["losses"], rtol=2e-5)
    np.testing.assert_allclose(norms, trace["grad_norms"], rtol=1e-4)
    for name, p in model.named_parameters():
        s, sq = trace["param_sum_sumsq"][name]
        got = p.detach().double()
        assert abs(float(got.pow(2).sum()) - sq) <= 1e-4 * sq, name
        scale = math.sqrt(sq * p.numel())
        assert abs(float(got.sum()) - s) <= 2e-4 * max(scale, 1e-12), name
