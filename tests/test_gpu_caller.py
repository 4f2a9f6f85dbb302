"""The caller of the boundary on the GPU: ``engine.backward`` and the gating.

minispeed's ``backward`` multiplies the loss by ``scale / gas``
(engine.py:227-233), autograd accumulates the micro-batch gradients in the
parameter dtype, and ``step`` runs the boundary only when the window closes
(engine.py:162-171, 254-266).  Three traces of minispeed training the
8 -> 32 -> 32 -> 1 MLP of its own tests (tests/common.py:19-32) through
autograd are replayed on the GPU through ``engine(x)`` /
``engine.backward`` / ``engine.step``:

* fp32 and bf16 at gas 2 (``mlp_fp32_trace``, ``mlp_bf16_trace``);
* fp16 at gas 3 with a dynamic loss scale starting at 2^20, window 2
  (``mlp_fp16_trace``): the factor scale / 3 rounds, the first six
  boundaries overflow and are skipped while the scale halves, then it grows
  back every two clean steps.

Per micro-batch, exactly: the loss and every accumulated ``param.grad``
equal those of a twin module on the same GPU whose loss is scaled by the
oracle's restatement of ``_scale_loss`` (same kernels, so bit for bit), and
``step()`` returns False until the window closes.  Per boundary: applied or
skipped, the loss-scale state, lr and step counts equal minispeed's record
exactly; the oracle started from the GPU's state with the GPU's gradients
gives the same decision, moments bit for bit and masters within 2 fp32 ulp.
Over the run: the losses, gradient norms and final parameters stay within
the trace tolerances of CPU-versus-GPU autograd (below), which only
reflect the different reduction orders of the forward/backward kernels.
"""

from __future__ import annotations

import copy
import types

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch import nn

import minispeed_amd as ms
from oracle import boundary as ob
from tests.golden_cases import DTYPES, META, MLP, arrays, scheduler_params
from tests.helpers import clip_override, master_step_within_ulps, step_hyper

pytestmark = pytest.mark.gpu
DEV = "cuda"

# CPU-versus-GPU autograd tolerances per trace (relative): losses, gradient
# norms, final fp32 masters.  fp32 differs only in reduction order; the
# half-precision forwards round their outputs to 8 / 11 significant bits.
# Measured on MI355X: fp32 2.2e-7 / 1.0e-7 / 1.2e-7, bf16 1.2e-3 / 1.7e-3 /
# 9.9e-3, fp16 4.0e-3 / 6.6e-4 / 9.6e-3 (a half gradient that differs in its
# last bit can move an Adam update by up to lr, here 1e-2, against masters of
# about 0.3).
TOL = {
    "mlp_fp32_trace": (1e-5, 1e-5, 1e-5),
    "mlp_bf16_trace": (5e-3, 5e-3, 3e-2),
    "mlp_fp16_trace": (5e-3, 5e-3, 3e-2),
}


def _bits(t: torch.Tensor) -> torch.Tensor:
    """Raw storage (an overflowing fp16 window holds inf/nan: compare bits)."""
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32)


def _oracle_for(case, arr, params):
    cfg = case["config"]
    opts = dict(cfg["optimizer"]["params"])
    opts["betas"] = tuple(opts["betas"])
    fp16 = cfg.get("fp16", {})
    ref_params = [nn.Parameter(torch.from_numpy(arr[f"init_p{i}"].copy())) for i in range(len(params))]
    ref = ob.Engine([ref_params], [opts], dtype=cfg["dtype"], zero_stage=0,
                    clip=cfg["gradient_clipping"], gas=case["gas"],
                    loss_scale=float(fp16.get("loss_scale", 0.0)),
                    initial_scale_power=int(fp16.get("initial_scale_power", 16)),
                    loss_scale_window=int(fp16.get("loss_scale_window", 1000)),
                    scheduler=cfg["scheduler"]["type"], scheduler_params=scheduler_params(cfg))
    return ref, ref_params


@pytest.mark.parametrize("name", ["mlp_fp32_trace", "mlp_bf16_trace", "mlp_fp16_trace"])
def test_backward_and_gating_replay_minispeeds_trace(name):
    case = META["cases"][name]
    arr = arrays(name)
    cfg = copy.deepcopy(case["config"])
    dtype = DTYPES[cfg["dtype"]]
    gas = case["gas"]
    model = MLP().to(DEV)
    with torch.no_grad():
        for i, p in enumerate(model.parameters()):
            p.copy_(torch.from_numpy(arr[f"init_p{i}"]))
    engine = ms.initialize(model=model, model_parameters=list(model.parameters()), config=cfg)
    params = list(model.parameters())
    twin = MLP().to(DEV).to(dtype)
    twin_params = list(twin.parameters())
    # the oracle's _scale_loss (engine.py:227-233) on a scaler kept in step
    # with the engine's
    scaler = ob.LossScaler(enabled=cfg["dtype"] == "fp16")
    holder = types.SimpleNamespace(scaler=scaler, gas=gas)
    ref, ref_params = _oracle_for(case, arr, params)
    g = engine.flat_groups[0]
    x = torch.from_numpy(arr["x"]).to(DEV)
    y = torch.from_numpy(arr["y"]).to(DEV)
    losses, boundaries = [], []
    for s in range(case["steps"]):
        with torch.no_grad():
            for tp, p in zip(twin_params, params):
                tp.copy_(p)
                tp.grad = None
        for mi in range(gas):
            loss = F.mse_loss(engine(x[s, mi]).float(), y[s, mi].float())
            losses.append(float(loss.detach()))
            engine.backward(loss)
            scaler.scale = engine.loss_scaler.scale
            twin_loss = F.mse_loss(twin(x[s, mi].to(dtype)).float(), y[s, mi].float())
            ob.Engine.scale_loss(holder, twin_loss).backward()
            assert torch.equal(twin_loss.detach(), loss.detach()), (s, mi)
            for k, (tp, p) in enumerate(zip(twin_params, params)):
                assert p.grad.dtype == dtype and _bits(p.grad).equal(_bits(tp.grad)), (s, mi, k)
            if mi < gas - 1:
                assert engine.step() is False            # window still open
                continue
            # the boundary, checked against the oracle from the GPU's state
            st = engine.optimizer.state[0]
            before = g.data.detach().cpu().clone()
            ref.load_state([before], [st["exp_avg"].cpu()], [st["exp_avg_sq"].cpu()], [st["step"]],
                           (engine.loss_scaler.scale, engine.loss_scaler.good_steps,
                            engine.loss_scaler.skipped_steps),
                           engine.lr_scheduler.last_epoch,
                           [pg["lr"] for pg in engine.optimizer.param_groups])
            for rp, p in zip(ref_params, params):
                rp.grad = p.grad.detach().cpu().clone()
            ref.micro_steps = engine.micro_steps
            hp = step_hyper(engine)
            applied = engine.step()
            assert engine.step() is False                # one update per boundary
            assert ref.step(clip_override=clip_override(engine) if applied else None) == applied
            assert all(p.grad is None for p in params)   # released at the boundary (flat.py:213)
            sc = engine.loss_scaler
            assert (sc.scale, sc.good_steps, sc.skipped_steps) == (
                ref.scaler.scale, ref.scaler.good_steps, ref.scaler.skipped_steps)
            if applied:
                assert abs(engine.grad_norm - ref.grad_norm) <= 1e-5 * ref.grad_norm
                np.testing.assert_array_equal(st["exp_avg"].cpu().numpy(),
                                              ref.state[0]["exp_avg"].numpy())
                np.testing.assert_array_equal(st["exp_avg_sq"].cpu().numpy(),
                                              ref.state[0]["exp_avg_sq"].numpy())
                ok, worst, nsq = master_step_within_ulps(
                    before.numpy(), g.data.cpu().numpy(), ref.groups[0].data.numpy(),
                    st["exp_avg"].cpu().numpy(), st["exp_avg_sq"].cpu().numpy(), **hp)
                assert ok, (s, worst, nsq)
            else:
                assert torch.equal(g.data.cpu(), before)
            boundaries.append({"applied": bool(applied), "scale": sc.scale,
                               "good_steps": sc.good_steps, "skipped_steps": sc.skipped_steps,
                               "grad_norm": engine.grad_norm,
                               "lr": [pg["lr"] for pg in engine.optimizer.param_groups],
                               "global_steps": engine.global_steps})

    # against minispeed's own CPU run
    rec = case["boundaries"]
    assert len(boundaries) == len(rec)
    exact = ("applied", "scale", "good_steps", "skipped_steps", "lr", "global_steps")
    for k, (got, want) in enumerate(zip(boundaries, rec)):
        assert {f: got[f] for f in exact} == {f: want[f] for f in exact}, k
    tl, tn, tp = TOL[name]
    worst_loss = float(np.max(np.abs(np.array(losses) - case["losses"]) / np.abs(case["losses"])))
    norms = [(b["grad_norm"], r["grad_norm"]) for b, r in zip(boundaries, rec) if r["grad_norm"]]
    worst_norm = max(abs(a - b) / b for a, b in norms)
    want = arr["final_master0"]
    worst_master = float(np.max(np.abs(g.data.cpu().numpy() - want)) / np.max(np.abs(want)))
    print(f"[{name}] worst relative deviation from minispeed's CPU run: loss {worst_loss:.3g}, "
          f"grad_norm {worst_norm:.3g}, final masters {worst_master:.3g}", flush=True)
    assert worst_loss <= tl and worst_norm <= tn and worst_master <= tp
    assert engine.global_steps == case["global_steps"]
