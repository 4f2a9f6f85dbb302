"""Parity at the benchmark workloads' real sizes.

* GPT-2-small buffer (124,439,808 params, 148 tensors), fp16 grads
  N(0,1e-3)*2^16, ZeRO-2, clip 1.0: each of the first steps checked against
  the oracle started from the GPU's state with the GPU's clip coefficient
  (moments bit-exact, masters within 2 ulp), then 100 boundaries with fresh
  seeded gradients against the oracle running on its own: every element of
  the masters and moments within 1e-5 of its largest magnitude along the
  run.
* 350M buffer (292 tensors), fp16, dynamic scale 2^16 with window 1000,
  inf/nan at 1-16 seeded positions of every 4th step for 200 steps: the
  skip / halve trajectory is bit-exact against the reference state machine
  and the masters, moments and model copy are untouched by skipped steps.
* 1.3B buffer (292 tensors), bf16 grads accumulated over 4 micro-batches by
  torch bf16 adds, ZeRO-1, WarmupDecayLR: the norm against a float64 sum of
  squares, a random million elements bit-exact against the kernel recipe,
  the fused and the materialized-flat-grad modes bitwise identical, two runs
  bitwise identical.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

import minispeed_amd as ms
from minispeed_amd.workloads import shapes_of
from oracle import boundary as ob
from oracle import recipe
from tests.helpers import clip_override, master_step_within_ulps, relative_within, step_hyper

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cfg(dtype, stage, *, clip=1.0, power=16, window=1000, sched=None, materialize=False, gas=1):
    cfg = {"train_micro_batch_size_per_gpu": 1, "gradient_accumulation_steps": gas,
           "gradient_clipping": clip, "dtype": dtype,
           "optimizer": {"type": "AdamW", "params": {"lr": 1e-3, "betas": [0.9, 0.999],
                                                      "eps": 1e-8, "weight_decay": 0.01}},
           "scheduler": sched or {"type": "WarmupLR", "params": {"warmup_num_steps": 0}},
           "zero_optimization": {"stage": stage}, "steps_per_print": 10 ** 9,
           "hip_boundary": {"materialize_flat_grad": materialize}}
    if dtype == "fp16":
        cfg["fp16"] = {"enabled": True, "loss_scale": 0, "initial_scale_power": power,
                       "loss_scale_window": window}
    return cfg


def _params(shapes, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    return [nn.Parameter(torch.randn(*s, generator=gen, device=DEV) * 0.02) for s in shapes]


def _engine(shapes, cfg, seed=0):
    params = _params(shapes, seed)
    mod = nn.ParameterList(params)
    return ms.initialize(model=mod, model_parameters=list(mod), config=cfg), params


class _Sample:
    """``count`` seeded flat indices of a group (unique, sorted) and the
    values of a ragged tensor list (gradients, parameters) there."""

    def __init__(self, g, count, seed):
        rng = np.random.default_rng(seed)
        offsets = np.array(g.layout.offsets, dtype=np.int64)
        self.idx = np.unique(rng.integers(0, g.numel, size=count))
        self.pi = np.searchsorted(offsets, self.idx, side="right") - 1
        self.local = self.idx - offsets[self.pi]
        self.idx_t = torch.from_numpy(self.idx).to(DEV)

    def gather(self, tensors, dtype=np.float32):
        """flat values of a ragged list at the sampled indices, on the CPU"""
        out = np.empty(len(self.idx), dtype=dtype)
        for k in np.unique(self.pi):
            sel = np.nonzero(self.pi == k)[0]
            t = tensors[k].detach().reshape(-1)[torch.from_numpy(self.local[sel]).to(DEV)].cpu()
            out[sel] = t.float().numpy() if dtype == np.float32 else t.view(torch.int16).numpy()
        return out


def _grads(shapes, dtype, gen, scale=1.0, std=1e-3):
    return [(torch.randn(*s, generator=gen, device=DEV) * (std * scale)).to(dtype) for s in shapes]


def test_gpt2_small_fp16_zero2_against_oracle():
    shapes = shapes_of("gpt2-124m")
    engine, params = _engine(shapes, _cfg("fp16", 2))
    ref_params = [nn.Parameter(p.detach().cpu().clone()) for p in params]
    ref = ob.Engine([ref_params], [{"lr": 1e-3, "betas": (0.9, 0.999), "eps": 1e-8,
                                    "weight_decay": 0.01}],
                    dtype="fp16", zero_stage=2, clip=1.0, initial_scale_power=16,
                    scheduler="WarmupLR", scheduler_params={"warmup_max_lr": 1e-3})
    gen = torch.Generator(device=DEV).manual_seed(42)
    g = engine.flat_groups[0]
    checked = 3
    for step in range(100):
        before = g.data.detach().cpu() if step < checked else None
        if step < checked:      # per-step check from the GPU's own state
            st = engine.optimizer.state[0]
            ref.load_state([before], [st["exp_avg"].cpu()], [st["exp_avg_sq"].cpu()], [st["step"]],
                           (engine.loss_scaler.scale, engine.loss_scaler.good_steps,
                            engine.loss_scaler.skipped_steps),
                           engine.lr_scheduler.last_epoch,
                           [pg["lr"] for pg in engine.optimizer.param_groups])
        grads = _grads(shapes, torch.float16, gen, scale=engine.loss_scaler.scale)
        for p, rp, gr in zip(params, ref_params, grads):
            p.grad = gr
            rp.grad = gr.cpu()
        engine.micro_steps += 1
        ref.micro_steps += 1
        hp = step_hyper(engine)
        assert engine.step() is True
        # per-step checks run the oracle's AdamW on the GPU's clip coefficient;
        # afterwards the oracle runs on its own (its own norms and coefficients)
        assert ref.step(clip_override=clip_override(engine) if step < checked else None) is True
        assert abs(engine.grad_norm - ref.grad_norm) <= 1e-5 * ref.grad_norm
        assert engine.loss_scaler.scale == ref.scaler.scale
        if step < checked:
            got = g.data.detach().cpu().numpy()
            want = ref.groups[0].data.numpy()
            ok, worst, nsq = master_step_within_ulps(
                before.numpy(), got, want, engine.optimizer.state[0]["exp_avg"].cpu().numpy(),
                engine.optimizer.state[0]["exp_avg_sq"].cpu().numpy(), **hp)
            print(f"[gpt2-124m] step {step}: masters within {worst:.2f} ulp of the oracle's; "
                  f"{nsq} elements further off where torch's CPU sqrt is not correctly rounded",
                  flush=True)
            assert ok, (step, worst, nsq)
            np.testing.assert_array_equal(engine.optimizer.state[0]["exp_avg"].cpu().numpy(),
                                          ref.state[0]["exp_avg"].numpy())
            np.testing.assert_array_equal(engine.optimizer.state[0]["exp_avg_sq"].cpu().numpy(),
                                          ref.state[0]["exp_avg_sq"].numpy())
            traj = [np.abs(x.numpy()).copy() for x in (ref.groups[0].data, ref.state[0]["exp_avg"],
                                                        ref.state[0]["exp_avg_sq"])]
        else:          # each element's largest magnitude along the oracle's trajectory
            for t, x in zip(traj, (ref.groups[0].data, ref.state[0]["exp_avg"],
                                   ref.state[0]["exp_avg_sq"])):
                np.maximum(t, np.abs(x.numpy()), out=t)
    # after 100 steps: 1e-5 relative per element, relative to the element's
    # largest magnitude along the run
    for name, got, want, t in (("master", g.data, ref.groups[0].data, traj[0]),
                               ("exp_avg", engine.optimizer.state[0]["exp_avg"], ref.state[0]["exp_avg"],
                                traj[1]),
                               ("exp_avg_sq", engine.optimizer.state[0]["exp_avg_sq"],
                                ref.state[0]["exp_avg_sq"], traj[2])):
        ok, worst = relative_within(got.detach().cpu().numpy(), want.numpy(), t)
        print(f"[gpt2-124m] after 100 steps, {name}: worst |diff| / bound = {worst:.3g}", flush=True)
        assert ok, (name, worst)
    assert engine.global_steps == 100 and not g.grad_shard.any()


def test_overflow_stress_350m_trajectory():
    shapes = shapes_of("gpt-350m")
    engine, params = _engine(shapes, _cfg("fp16", 0))
    sizes = [int(np.prod(s)) for s in shapes]
    rng = np.random.default_rng(1234)
    scaler = ob.LossScaler(True, 0.0, 1000)
    scaler.set_scale_from_power(16)
    gen = torch.Generator(device=DEV).manual_seed(7)
    g = engine.flat_groups[0]
    specials = [float("inf"), float("-inf"), float("nan")]
    skipped = 0
    # applied steps checked bit for bit against the kernels' recipe on 2^18
    # sampled elements: the first ones, the ones right after an injected
    # overflow (the scale just halved), and the last ones (scale 1)
    checked = {0, 1, 4, 8, 100, 196, 197, 198}
    sample = _Sample(g, 1 << 18, seed=5)
    for step in range(200):
        grads = _grads(shapes, torch.float16, gen, scale=engine.loss_scaler.scale)
        inject = step % 4 == 3
        if inject:
            for _ in range(int(rng.integers(1, 17))):
                ti = int(rng.integers(0, len(shapes)))
                grads[ti].view(-1)[int(rng.integers(0, sizes[ti]))] = specials[int(rng.integers(0, 3))]
            state0 = (g.data.clone(), engine.optimizer.state[0]["exp_avg"].clone(),
                      engine.optimizer.state[0]["exp_avg_sq"].clone(), params[5].detach().clone())
        if step in checked:
            assert not inject
            it = sample.idx_t
            p0, m0, v0 = (x[it].cpu().numpy() for x in (g.data, engine.optimizer.state[0]["exp_avg"],
                                                       engine.optimizer.state[0]["exp_avg_sq"]))
            g_s = sample.gather(grads)
            lr = engine.optimizer.param_groups[0]["lr"]
            t_adam = engine.optimizer.state[0]["step"] + 1
            scale_before = engine.loss_scaler.scale
        for p, gr in zip(params, grads):
            p.grad = gr
        engine.micro_steps += 1
        applied = engine.step()
        if step in checked:
            sc = engine.last_boundary
            wp, wm, wv = recipe.adamw_step(p0, m0, v0, g_s, lr=lr, betas=(0.9, 0.999), eps=1e-8,
                                           wd=0.01, step=t_adam, grad_scale=scale_before,
                                           unscale=scale_before != 1.0,
                                           clip_coef=float(np.float32(sc.coef)) if sc.clip_applied else None)
            for got, want in ((g.data, wp), (engine.optimizer.state[0]["exp_avg"], wm),
                              (engine.optimizer.state[0]["exp_avg_sq"], wv)):
                np.testing.assert_array_equal(got[it].cpu().numpy().view(np.int32), want.view(np.int32),
                                              err_msg=str(step))
            np.testing.assert_array_equal(sample.gather(params, np.int16),
                                          torch.from_numpy(wp).half().view(torch.int16).numpy())
        scaler.update(overflow=inject)
        skipped += inject
        assert applied == (not inject), step
        assert (engine.loss_scaler.scale, engine.loss_scaler.good_steps,
                engine.loss_scaler.skipped_steps) == (scaler.scale, scaler.good_steps,
                                                      scaler.skipped_steps), step
        if inject:
            assert torch.equal(g.data, state0[0])
            assert torch.equal(engine.optimizer.state[0]["exp_avg"], state0[1])
            assert torch.equal(engine.optimizer.state[0]["exp_avg_sq"], state0[2])
            assert torch.equal(params[5].detach(), state0[3])
    assert engine.skipped_steps == skipped == 50
    assert engine.global_steps == 150 and engine.loss_scaler.scale == 1.0


def _bf16_gas4_grads(shapes, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    acc = None
    for _ in range(4):
        micro = _grads(shapes, torch.bfloat16, gen, std=1e-3)
        if acc is None:
            acc = micro
        else:
            for a, m in zip(acc, micro):
                a.add_(m)              # autograd's accumulation into .grad (bf16)
    return acc


def test_1p3b_bf16_gas4_norm_sampled_elements_and_modes():
    shapes = shapes_of("gpt-1.3b")
    sched = {"type": "WarmupDecayLR", "params": {"warmup_min_lr": 0.0, "warmup_max_lr": 1e-3,
                                                  "warmup_num_steps": 100, "total_num_steps": 1000}}
    engine, params = _engine(shapes, _cfg("bf16", 1, sched=sched, gas=4), seed=3)
    g = engine.flat_groups[0]
    sample = _Sample(g, 1_000_000, seed=0)
    idx, idx_t, gather = sample.idx, sample.idx_t, sample.gather

    for step in range(2):
        grads = _bf16_gas4_grads(shapes, seed=10 + step)
        p0 = g.data[idx_t].cpu().numpy()
        m0 = engine.optimizer.state[0]["exp_avg"][idx_t].cpu().numpy()
        v0 = engine.optimizer.state[0]["exp_avg_sq"][idx_t].cpu().numpy()
        g_s = gather(grads)
        exact = sum(float(t.double().pow(2).sum()) for t in grads)
        lr = engine.optimizer.param_groups[0]["lr"]
        t_adam = engine.optimizer.state[0]["step"] + 1
        for p, gr in zip(params, grads):
            p.grad = gr
        engine.micro_steps += 4
        assert engine.step() is True
        sc = engine.last_boundary
        assert abs(int(np.float32(sc.sumsq).view(np.int32)) - int(np.float32(exact).view(np.int32))) <= 1
        assert abs(engine.grad_norm - np.sqrt(exact)) <= 1e-6 * np.sqrt(exact)
        assert sc.clip_applied == 1
        wp, wm, wv = recipe.adamw_step(p0, m0, v0, g_s, lr=lr, betas=(0.9, 0.999), eps=1e-8,
                                       wd=0.01, step=t_adam, clip_coef=float(np.float32(sc.coef)))
        np.testing.assert_array_equal(g.data[idx_t].cpu().numpy().view(np.int32), wp.view(np.int32))
        np.testing.assert_array_equal(engine.optimizer.state[0]["exp_avg"][idx_t].cpu().numpy(), wm)
        np.testing.assert_array_equal(engine.optimizer.state[0]["exp_avg_sq"][idx_t].cpu().numpy(), wv)
        model = gather(params)
        np.testing.assert_array_equal(model, torch.from_numpy(wp).to(torch.bfloat16).float().numpy())
        del grads

    # fused vs materialized flat grad, and run-to-run determinism, from one state
    state = (g.data.clone(), engine.optimizer.state[0]["exp_avg"].clone(),
             engine.optimizer.state[0]["exp_avg_sq"].clone())
    lr0, epoch0 = engine.optimizer.param_groups[0]["lr"], engine.lr_scheduler.last_epoch
    results = []
    for materialize in (False, True, False):
        engine.config.materialize_flat_grad = materialize
        g.data.copy_(state[0])
        engine.optimizer.state[0]["exp_avg"].copy_(state[1])
        engine.optimizer.state[0]["exp_avg_sq"].copy_(state[2])
        engine.optimizer.state[0]["step"] = 2
        engine.optimizer.param_groups[0]["lr"] = lr0      # the schedule advances per step
        engine.lr_scheduler.last_epoch = epoch0
        for p, gr in zip(params, _bf16_gas4_grads(shapes, seed=99)):
            p.grad = gr
        engine.micro_steps += 4
        assert engine.step() is True
        results.append((engine.last_boundary.sumsq, g.data.clone(),
                        engine.optimizer.state[0]["exp_avg_sq"].clone(), params[7].detach().clone()))
        if materialize:
            assert not g.grad.any()
    for other in results[1:]:
        assert other[0] == results[0][0]
        assert torch.equal(other[1], results[0][1]) and torch.equal(other[2], results[0][2])
        assert torch.equal(other[3].view(torch.int16), results[0][3].view(torch.int16))


def test_one_rank_shard_step_and_cast_on_gather():
    """One rank's 1/8 ZeRO-3 share (rank 5 of 8) of the GPT-2-small list at
    component level: K1 -> K2 -> K3 over the owned range with ragged bf16
    gradient pieces and placeholder cast targets, every element against the
    kernel recipe; then the cast-on-gather of a full fp32 buffer into the
    full-shaped parameters, bit-exact against round-to-nearest-even."""
    import ctypes

    from minispeed_amd import _native
    from minispeed_amd.boundary import adamw_params
    from minispeed_amd.flat import FlatLayout, check_table

    lib = _native.load()
    shapes = shapes_of("gpt2-124m")
    numels = [int(np.prod(s)) for s in shapes]
    lay = FlatLayout(numels, rank=5, world_size=8, zero_stage=3)
    lo, hi = lay.shard_start, lay.shard_end
    S, N = hi - lo, lay.numel_padded
    gen = torch.Generator(device=DEV).manual_seed(11)
    grad = (torch.randn(S, generator=gen, device=DEV) * 1e-4).to(torch.bfloat16)
    holder = torch.zeros(S, dtype=torch.bfloat16, device=DEV)
    master = torch.randn(S, generator=gen, device=DEV) * 0.02
    m = torch.randn(S, generator=gen, device=DEV) * 1e-5
    v = torch.rand(S, generator=gen, device=DEV) * 1e-9
    p0, m0, v0, g0 = (t.cpu().numpy().copy() for t in (master, m, v, grad.float()))
    gs, ms_ = [], []
    for off, n in zip(lay.offsets, numels):
        a, b = max(off, lo), min(off + n, hi)
        gs.append((grad.data_ptr() + (a - lo) * 2, (a, b), 2) if b > a else None)
        ms_.append((holder.data_ptr() + (a - lo) * 2, (a, b), 2) if b > a else None)
    table = lay.segments(lo, hi, gs, ms_)
    check_table(table, lo, hi)
    tdev = torch.from_numpy(table).to(DEV)
    nb = _native.stats_blocks()
    psum = torch.empty(nb, dtype=torch.float64, device=DEV)
    pflag = torch.empty(nb, dtype=torch.int32, device=DEV)
    nt = _native.scan_tiles(hi - lo)
    tsum = torch.empty(nt, dtype=torch.float64, device=DEV)
    tflag = torch.empty(nt, dtype=torch.int32, device=DEV)
    scal = torch.empty(_native.SCALARS_BYTES, dtype=torch.uint8, device=DEV)
    st = _native.stream_handle(torch.device(DEV))
    _native.check(lib.ms_grad_stats(tdev.data_ptr(), len(table), _native.DTYPE_BF16, lo, hi, lo, hi,
                                    0, 1.0, None, tsum.data_ptr(), tflag.data_ptr(), nt,
                                    psum.data_ptr(), pflag.data_ptr(), nb, st), "k1")
    _native.check(lib.ms_norm_clip(psum.data_ptr(), pflag.data_ptr(), nb, 1, 1, 0.05, 0, 1.0, 0, 0,
                                   1000, 1.0, 2.0 ** 24, scal.data_ptr(), None, st), "k2")
    hp = adamw_params(1e-3, (0.9, 0.999), 1e-8, 0.01, 4)
    _native.check(lib.ms_fused_adamw(master.data_ptr(), m.data_ptr(), v.data_ptr(), None,
                                     tdev.data_ptr(), len(table), _native.DTYPE_BF16,
                                     _native.DTYPE_BF16, lo, hi, ctypes.byref(hp),
                                     scal.data_ptr(), st), "k3")
    torch.cuda.synchronize()
    sc = _native.StepScalars.from_buffer_copy(scal.cpu().numpy().tobytes())
    exact = recipe.sumsq_f64(g0)
    assert not sc.overflow and sc.clip_applied
    assert abs(int(np.float32(sc.sumsq).view(np.int32)) - int(np.float32(exact).view(np.int32))) <= 1
    wp, wm, wv = recipe.adamw_step(p0, m0, v0, g0, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, wd=0.01,
                                   step=4, clip_coef=float(np.float32(sc.coef)))
    np.testing.assert_array_equal(master.cpu().numpy().view(np.int32), wp.view(np.int32))
    np.testing.assert_array_equal(m.cpu().numpy().view(np.int32), wm.view(np.int32))
    np.testing.assert_array_equal(v.cpu().numpy().view(np.int32), wv.view(np.int32))
    assert torch.equal(holder.view(torch.int16),
                       torch.from_numpy(wp).to(torch.bfloat16).to(DEV).view(torch.int16))

    full = torch.randn(N, generator=gen, device=DEV) * 0.02
    full[:5] = torch.tensor([3.0e38, -1e-40, 0.0, -0.0, 1.00390625], device=DEV)
    params16 = [torch.empty(s, dtype=torch.bfloat16, device=DEV) for s in shapes]
    gtable = lay.segments(0, N, [None] * len(numels),
                          [(t.data_ptr(), (off, off + t.numel()), 2) for t, off in zip(params16, lay.offsets)])
    check_table(gtable, 0, N)
    gdev = torch.from_numpy(gtable).to(DEV)
    _native.check(lib.ms_cast_to_model(full.data_ptr(), 0, N, gdev.data_ptr(), len(gtable),
                                       _native.DTYPE_BF16, st), "k4")
    torch.cuda.synchronize()
    want = full[:lay.numel].to(torch.bfloat16)
    got = torch.cat([t.reshape(-1) for t in params16])
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_llama3_8b_whole_model_one_rank_flat_indices_beyond_2_32():
    """All of Llama-3-8B (8,030,261,248 params, 291 tensors) as one group at
    world size 1, bf16, ZeRO-3: the flat indices run past 2^32, so every
    index computation of the kernels is exercised in 64 bits.  One
    boundary: the norm against a float64 sum of squares, a million random
    elements (about half beyond 2^32) bit-exact against the kernel recipe,
    the bf16 model copy the round-to-nearest-even cast of the masters."""
    shapes = shapes_of("llama3-8b")
    gen = torch.Generator(device=DEV).manual_seed(21)
    params = [nn.Parameter((torch.randn(*s, generator=gen, device=DEV) * 0.02).to(torch.bfloat16))
              for s in shapes]
    mod = nn.ParameterList(params)
    engine = ms.initialize(model=mod, model_parameters=list(mod), config=_cfg("bf16", 3))
    g = engine.flat_groups[0]
    n = g.numel
    assert n == 8_030_261_248 and n > 2 ** 32 and g.whole_range
    offsets = np.array(g.layout.offsets, dtype=np.int64)
    rng = np.random.default_rng(1)
    idx = np.unique(np.concatenate([rng.integers(0, n, size=1_000_000),
                                    np.array([0, 2 ** 32 - 1, 2 ** 32, 2 ** 32 + 1, n - 1])]))
    assert (idx >= 2 ** 32).sum() > 400_000
    pi = np.searchsorted(offsets, idx, side="right") - 1
    local = idx - offsets[pi]
    idx_t = torch.from_numpy(idx).to(DEV)

    def gather(tensors):
        out = np.empty(len(idx), dtype=np.float32)
        for k in np.unique(pi):
            sel = np.nonzero(pi == k)[0]
            t = tensors[k].detach().reshape(-1)
            out[sel] = t[torch.from_numpy(local[sel]).to(DEV)].float().cpu().numpy()
        return out

    engine.optimizer.gather_parameters()               # what the forward does
    grads = _grads(shapes, torch.bfloat16, gen, std=1e-4)
    p0 = g.data[idx_t].cpu().numpy()
    m0 = engine.optimizer.state[0]["exp_avg"][idx_t].cpu().numpy()
    v0 = engine.optimizer.state[0]["exp_avg_sq"][idx_t].cpu().numpy()
    g_s = gather(grads)
    exact = sum(float(t.double().pow(2).sum()) for t in grads)
    for p, gr in zip(params, grads):
        p.grad = gr
    del grads
    engine.micro_steps += 1
    assert engine.step() is True
    sc = engine.last_boundary
    assert not sc.overflow and sc.clip_applied == 1
    assert abs(engine.grad_norm - np.sqrt(exact)) <= 1e-6 * np.sqrt(exact)
    wp, wm, wv = recipe.adamw_step(p0, m0, v0, g_s, lr=1e-3, betas=(0.9, 0.999), eps=1e-8,
                                   wd=0.01, step=1, clip_coef=float(np.float32(sc.coef)))
    np.testing.assert_array_equal(g.data[idx_t].cpu().numpy().view(np.int32), wp.view(np.int32))
    np.testing.assert_array_equal(engine.optimizer.state[0]["exp_avg"][idx_t].cpu().numpy(), wm)
    np.testing.assert_array_equal(engine.optimizer.state[0]["exp_avg_sq"][idx_t].cpu().numpy(), wv)
    assert not engine.optimizer.params_gathered
    model = gather(params)                              # the freed placeholders
    np.testing.assert_array_equal(model, torch.from_numpy(wp).to(torch.bfloat16).float().numpy())


def test_llama3_8b_rank3_of_8_shard_at_its_exact_geometry():
    """One rank's 1/8 ZeRO-3 shard of Llama-3-8B at its real geometry: rank 3
    of 8 owns [3,011,347,968, 4,015,130,624) of the 8,030,261,248-element
    flat space, a table of ragged pieces whose first and last cut tensors
    mid-way.  K1 -> K2 -> K3 over that table with bf16 gradient pieces
    N(0,1e-4) and bf16 placeholder cast targets: the sum of squares within 1
    fp32 ulp of a float64 sum over all 1,003,782,656 elements, a million
    sampled elements (plus every piece edge) bit-exact against the kernel
    recipe with the GPU's clip coefficient, the placeholders the
    round-to-nearest-even cast of the masters.  Then the cast-on-gather of
    a full fp32 master buffer into the 291 full-shaped bf16 parameters (K4),
    a million sampled elements (plus every tensor edge) bit-exact against
    torch's cast."""
    import ctypes

    from minispeed_amd import _native
    from minispeed_amd.boundary import adamw_params
    from minispeed_amd.flat import FlatLayout, check_table

    lib = _native.load()
    shapes = shapes_of("llama3-8b")
    numels = [int(np.prod(s)) for s in shapes]
    lay = FlatLayout(numels, rank=3, world_size=8, zero_stage=3)
    lo, hi = lay.shard_start, lay.shard_end
    S, N = hi - lo, lay.numel_padded
    assert (lo, hi, N) == (3_011_347_968, 4_015_130_624, 8_030_261_248)
    print(f"[llama3-8b shard] rank 3 of 8: [{lo:,}, {hi:,}), {S:,} elements", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(31)
    grad = torch.empty(S, dtype=torch.bfloat16, device=DEV)
    master = torch.empty(S, device=DEV)
    m = torch.empty(S, device=DEV)
    v = torch.empty(S, device=DEV)
    chunk = 1 << 27
    exact = 0.0
    for a in range(0, S, chunk):      # bounded fp32 / fp64 temporaries
        b = min(S, a + chunk)
        grad[a:b] = torch.randn(b - a, generator=gen, device=DEV) * 1e-4
        exact += float(grad[a:b].double().pow(2).sum())
        master[a:b] = torch.randn(b - a, generator=gen, device=DEV) * 0.02
        m[a:b] = torch.randn(b - a, generator=gen, device=DEV) * 1e-5
        v[a:b] = torch.rand(b - a, generator=gen, device=DEV) * 1e-9
    holder = torch.zeros(S, dtype=torch.bfloat16, device=DEV)
    gs, ms_ = [], []
    for off, n in zip(lay.offsets, numels):
        a, b = max(off, lo), min(off + n, hi)
        gs.append((grad.data_ptr() + (a - lo) * 2, (a, b), 2) if b > a else None)
        ms_.append((holder.data_ptr() + (a - lo) * 2, (a, b), 2) if b > a else None)
    table = lay.segments(lo, hi, gs, ms_)
    check_table(table, lo, hi)
    pieces = len(table)
    assert pieces == 42 and table[0, 0] == lo and table[0, 0] % 1024 != 0
    edges = np.concatenate([table[:, 0], table[:, 0] + table[:, 1] - 1, table[:, 0] + 1]) - lo
    rng = np.random.default_rng(3)
    idx = np.unique(np.concatenate([rng.integers(0, S, size=1_000_000), edges[edges < S]]))
    idx_t = torch.from_numpy(idx).to(DEV)
    p0, m0, v0 = (t[idx_t].cpu().numpy() for t in (master, m, v))
    g0 = grad[idx_t].float().cpu().numpy()
    tdev = torch.from_numpy(table).to(DEV)
    nb = _native.stats_blocks()
    psum = torch.empty(nb, dtype=torch.float64, device=DEV)
    pflag = torch.empty(nb, dtype=torch.int32, device=DEV)
    nt = _native.scan_tiles(hi - lo)
    tsum = torch.empty(nt, dtype=torch.float64, device=DEV)
    tflag = torch.empty(nt, dtype=torch.int32, device=DEV)
    scal = torch.empty(_native.SCALARS_BYTES, dtype=torch.uint8, device=DEV)
    st = _native.stream_handle(torch.device(DEV))
    _native.check(lib.ms_grad_stats(tdev.data_ptr(), pieces, _native.DTYPE_BF16, lo, hi, lo, hi,
                                    0, 1.0, None, tsum.data_ptr(), tflag.data_ptr(), nt,
                                    psum.data_ptr(), pflag.data_ptr(), nb, st), "k1")
    _native.check(lib.ms_norm_clip(psum.data_ptr(), pflag.data_ptr(), nb, 1, 1, 1.0, 0, 1.0, 0, 0,
                                   1000, 1.0, 2.0 ** 24, scal.data_ptr(), None, st), "k2")
    hp = adamw_params(1e-3, (0.9, 0.999), 1e-8, 0.01, 3)
    _native.check(lib.ms_fused_adamw(master.data_ptr(), m.data_ptr(), v.data_ptr(), None,
                                     tdev.data_ptr(), pieces, _native.DTYPE_BF16,
                                     _native.DTYPE_BF16, lo, hi, ctypes.byref(hp),
                                     scal.data_ptr(), st), "k3")
    torch.cuda.synchronize()
    sc = _native.StepScalars.from_buffer_copy(scal.cpu().numpy().tobytes())
    assert not sc.overflow and sc.clip_applied        # norm ~ sqrt(1e9 * 1e-8) ~ 3.2 > 1
    assert abs(int(np.float32(sc.sumsq).view(np.int32)) - int(np.float32(exact).view(np.int32))) <= 1
    wp, wm, wv = recipe.adamw_step(p0, m0, v0, g0, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, wd=0.01,
                                   step=3, clip_coef=float(np.float32(sc.coef)))
    np.testing.assert_array_equal(master[idx_t].cpu().numpy().view(np.int32), wp.view(np.int32))
    np.testing.assert_array_equal(m[idx_t].cpu().numpy().view(np.int32), wm.view(np.int32))
    np.testing.assert_array_equal(v[idx_t].cpu().numpy().view(np.int32), wv.view(np.int32))
    assert torch.equal(holder[idx_t].cpu().view(torch.int16),
                       torch.from_numpy(wp).to(torch.bfloat16).view(torch.int16))
    del grad, holder, master, m, v, tdev
    torch.cuda.empty_cache()

    print(f"[llama3-8b shard] cast-on-gather of {N:,} fp32 masters", flush=True)
    full = torch.empty(N, device=DEV)
    for a in range(0, N, chunk):
        b = min(N, a + chunk)
        full[a:b] = torch.randn(b - a, generator=gen, device=DEV) * 0.02
    params16 = torch.empty(N, dtype=torch.bfloat16, device=DEV)
    gtable = lay.segments(0, N, [None] * len(numels),
                          [(params16.data_ptr() + off * 2, (off, off + n), 2)
                           for off, n in zip(lay.offsets, numels)])
    check_table(gtable, 0, N)
    gdev = torch.from_numpy(gtable).to(DEV)
    _native.check(lib.ms_cast_to_model(full.data_ptr(), 0, N, gdev.data_ptr(), len(gtable),
                                       _native.DTYPE_BF16, st), "k4")
    torch.cuda.synchronize()
    starts = np.array(lay.offsets, dtype=np.int64)
    ends = starts + np.array(numels, dtype=np.int64) - 1
    sample = np.unique(np.concatenate([rng.integers(0, N, size=1_000_000), starts, ends]))
    s_t = torch.from_numpy(sample).to(DEV)
    assert torch.equal(params16[s_t].view(torch.int16), full[s_t].to(torch.bfloat16).view(torch.int16))
