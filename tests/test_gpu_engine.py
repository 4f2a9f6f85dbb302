"""Engine behaviour on the GPU, the properties minispeed's own test suite
asserts (tests/test_engine.py, tests/test_gpu.py, tests/test_zero3.py),
with the boundary step running as the HIP kernels."""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch import nn

import minispeed_amd as ms
from minispeed_amd.flat import FlatParamGroup
from minispeed_amd.precision import has_overflow

pytestmark = pytest.mark.gpu
DEV = "cuda"
STEPS, GAS, MICRO = 6, 2, 4


class MLP(nn.Module):
    def __init__(self):
        super().__init__()
        self.net = nn.Sequential(nn.Linear(8, 32), nn.Tanh(), nn.Linear(32, 32), nn.ReLU(),
                                 nn.LayerNorm(32), nn.Linear(32, 1))

    def forward(self, x):
        return self.net(x)


def build_model(seed=1234):
    torch.manual_seed(seed)
    return MLP().to(DEV)


def make_batch(steps, gas, micro, seed=7):
    g = torch.Generator().manual_seed(seed)
    n = steps * gas * micro
    x = torch.randn(n, 8, generator=g).view(steps, gas, micro, 8)
    y = torch.randn(n, 1, generator=g).view(steps, gas, micro, 1)
    return x.to(DEV), y.to(DEV)


def config(micro=MICRO, gas=GAS, lr=1e-3, wd=0.01, clip=1.0, dtype="fp32", stage=0,
           warmup=0, total=None, scheduler="WarmupLR", power=8, window=100, materialize=False):
    sp = {"warmup_min_lr": 0.0, "warmup_max_lr": lr, "warmup_num_steps": warmup}
    if total is not None:
        sp["total_num_steps"] = total
    cfg = {"train_micro_batch_size_per_gpu": micro, "gradient_accumulation_steps": gas,
           "gradient_clipping": clip, "dtype": dtype,
           "optimizer": {"type": "AdamW", "params": {"lr": lr, "betas": [0.9, 0.999], "eps": 1e-8,
                                                      "weight_decay": wd}},
           "scheduler": {"type": scheduler, "params": sp},
           "zero_optimization": {"stage": stage}, "steps_per_print": 1000,
           "hip_boundary": {"materialize_flat_grad": materialize}}
    if dtype == "fp16":
        cfg["fp16"] = {"enabled": True, "loss_scale": 0, "initial_scale_power": power,
                       "loss_scale_window": window}
    elif dtype == "bf16":
        cfg["bf16"] = {"enabled": True}
    return cfg


def mse(pred, y):
    return F.mse_loss(pred.float(), y.float())


def train(engine, x, y, steps, gas):
    losses = []
    engine.train()
    for s in range(steps):
        for m in range(gas):
            loss = mse(engine(x[s, m]), y[s, m])
            losses.append(float(loss.detach()))
            engine.backward(loss)
            engine.step()
    return losses


def test_engine_matches_textbook_adamw_with_clipping():
    """minispeed tests/test_engine.py:45-64: engine == torch.optim.AdamW +
    clip_grad_norm_ at rtol 1e-4."""
    lr, wd, clip = 1e-3, 0.01, 1.0
    x, y = make_batch(STEPS, GAS, MICRO)
    ref = build_model()
    opt = torch.optim.AdamW(ref.parameters(), lr=lr, betas=(0.9, 0.999), eps=1e-8, weight_decay=wd)
    ref_losses = []
    for s in range(STEPS):
        for m in range(GAS):
            loss = F.mse_loss(ref(x[s, m]), y[s, m]) / GAS
            ref_losses.append(float(loss.detach()) * GAS)
            loss.backward()
        torch.nn.utils.clip_grad_norm_(ref.parameters(), clip)
        opt.step()
        opt.zero_grad(set_to_none=True)
    model = build_model()
    engine = ms.initialize(model=model, model_parameters=list(model.parameters()),
                           config=config(lr=lr, wd=wd, clip=clip))
    losses = train(engine, x, y, STEPS, GAS)
    assert engine.global_steps == STEPS
    np.testing.assert_allclose(losses, ref_losses, rtol=1e-4, atol=1e-6)
    for a, b in zip(model.parameters(), ref.parameters()):
        torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-6)


def test_gradient_accumulation_equals_large_batch():
    x, y = make_batch(STEPS, GAS, MICRO)
    big = build_model()
    e_big = ms.initialize(model=big, model_parameters=list(big.parameters()),
                          config=config(micro=MICRO * GAS, gas=1, lr=5e-3, wd=0.0, clip=None))
    train(e_big, x.reshape(STEPS, 1, GAS * MICRO, 8), y.reshape(STEPS, 1, GAS * MICRO, 1), STEPS, 1)
    acc = build_model()
    e_acc = ms.initialize(model=acc, model_parameters=list(acc.parameters()),
                          config=config(lr=5e-3, wd=0.0, clip=None))
    train(e_acc, x, y, STEPS, GAS)
    for a, b in zip(acc.parameters(), big.parameters()):
        torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-6)


def test_step_applies_once_per_boundary_and_tuple_unpacking():
    model = build_model()
    engine, optimizer, none, sched = ms.initialize(model=model, model_parameters=list(model.parameters()),
                                                   config=config())
    assert optimizer is engine.optimizer and sched is engine.lr_scheduler and none is None
    x, y = make_batch(1, GAS, MICRO)
    applied = []
    for m in range(GAS):
        engine.backward(mse(engine(x[0, m]), y[0, m]))
        applied.append(engine.step())
        assert engine.is_gradient_accumulation_boundary == (m == GAS - 1)
    assert applied == [False, True]
    assert engine.step() is False and engine.global_steps == 1
    assert all(p.grad is None for p in model.parameters())     # released at the boundary


def test_bf16_learns_with_fp32_masters():
    x, y = make_batch(STEPS, GAS, MICRO)
    model = build_model()
    engine = ms.initialize(model=model, model_parameters=list(model.parameters()),
                           config=config(dtype="bf16", lr=1e-2, clip=None))
    losses = train(engine, x, y, STEPS, GAS)
    assert np.all(np.isfinite(losses)) and losses[-1] < losses[0]
    assert next(model.parameters()).dtype == torch.bfloat16
    assert engine.flat_groups[0].data.dtype == torch.float32
    assert engine.get_loss_scale() == 1.0
    for (off, p), n in zip(engine.flat_groups[0]._offsets, engine.flat_groups[0]._numels):
        want = engine.flat_groups[0].data[off:off + n].to(torch.bfloat16).view(p.shape)
        assert torch.equal(p.data.view(torch.int16), want.view(torch.int16))


def test_fp16_trains_and_scale_grows():
    x, y = make_batch(STEPS, GAS, MICRO)
    model = build_model()
    engine = ms.initialize(model=model, model_parameters=list(model.parameters()),
                           config=config(dtype="fp16", power=4, window=3, lr=1e-2, clip=1.0))
    losses = train(engine, x, y, STEPS, GAS)
    assert np.all(np.isfinite(losses)) and losses[-1] < losses[0]
    assert next(model.parameters()).dtype == torch.float16
    assert engine.get_loss_scale() > 2.0 ** 4 and engine.loss_scaler.skipped_steps == 0
    assert engine.grad_norm is not None and engine.grad_norm > 0


@pytest.mark.parametrize("stage", [0, 2, 3])
def test_fp16_forced_inf_skips_step(stage):
    """minispeed tests/test_gpu.py:51-89 and tests/test_zero3.py:184-210."""
    x, y = make_batch(STEPS + 2, GAS, MICRO)
    model = build_model()
    engine = ms.initialize(model=model, model_parameters=list(model.parameters()),
                           config=config(dtype="fp16", power=6, lr=1e-2, clip=1.0, warmup=5,
                                         stage=stage))
    train(engine, x, y, 1, GAS)
    for m in range(GAS):
        engine.backward(mse(engine(x[1, m]), y[1, m]))
    for p in model.parameters():
        if p.grad is not None and p.grad.numel():
            p.grad.reshape(-1)[0] = float("inf")
            break
    steps0, scale0, lr0 = engine.global_steps, engine.get_loss_scale(), engine.lr_scheduler.get_last_lr()
    masters0 = engine.flat_groups[0].data.clone()
    moments0 = [st["exp_avg"].clone() for st in engine.optimizer.state]
    before = {n: p.detach().clone() for n, p in model.named_parameters()}
    assert engine.step() is False
    assert engine.global_steps == steps0 and engine.skipped_steps == 1
    assert engine.get_loss_scale() == scale0 / 2
    assert engine.lr_scheduler.get_last_lr() == lr0
    assert torch.equal(engine.flat_groups[0].data, masters0)
    assert all(torch.equal(a["exp_avg"], b) for a, b in zip(engine.optimizer.state, moments0))
    assert [st["step"] for st in engine.optimizer.state] == [steps0]
    if stage < 3:
        for n, p in model.named_parameters():
            assert torch.equal(p.view(torch.int16), before[n].view(torch.int16))
    else:
        assert not engine.optimizer.params_gathered
        assert engine.flat_groups[0].grad is None
    losses = train(engine, x[2:], y[2:], 2, GAS)
    assert np.all(np.isfinite(losses)) and engine.global_steps == steps0 + 2


def test_stage3_matches_stage0():
    x, y = make_batch(4, GAS, MICRO)
    out = {}
    for stage in (0, 3):
        model = build_model()
        engine = ms.initialize(model=model, model_parameters=list(model.parameters()),
                               config=config(stage=stage))
        losses = train(engine, x, y, 4, GAS)
        out[stage] = (losses, {k: v.clone() for k, v in engine.state_dict().items()}, engine)
    np.testing.assert_allclose(out[3][0], out[0][0], rtol=1e-5, atol=1e-7)
    for k, v in out[0][1].items():
        torch.testing.assert_close(out[3][1][k], v, rtol=1e-5, atol=1e-7)
    assert out[3][2].global_steps == out[0][2].global_steps == 4


def test_stage3_lifecycle():
    """minispeed tests/test_zero3.py:51-91."""
    x, y = make_batch(1, GAS, MICRO)
    model = build_model()
    engine = ms.initialize(model=model, model_parameters=list(model.parameters()),
                           config=config(stage=3))
    g = engine.flat_groups[0]
    shapes = [p.shape for p in build_model().parameters()]
    assert not engine.optimizer.params_gathered
    assert all(p.data.dim() == 1 for p in model.parameters()) and g.grad is None
    loss = mse(engine(x[0, 0]), y[0, 0])
    assert engine.optimizer.params_gathered
    assert [p.shape for p in model.parameters()] == shapes
    engine.backward(loss)
    assert engine.step() is False and engine.optimizer.params_gathered
    engine.backward(mse(engine(x[0, 1]), y[0, 1]))
    assert engine.step() is True
    assert not engine.optimizer.params_gathered
    assert all(p.data.dim() == 1 for p in model.parameters())
    assert g.grad is None and g.data.numel() == g.numel_shard()
    assert engine.optimizer.state[0]["exp_avg"].numel() == g.numel_shard()
    raw = model.state_dict()
    full = engine.state_dict()
    for k in full:
        assert raw[k].dim() == 1 and full[k].shape.numel() == raw[k].numel()
    engine.eval()
    with torch.no_grad():
        assert engine(x[0, 0]).shape == (MICRO, 1)


def test_stage3_partition_roundtrip_as_one_rank_of_two():
    """minispeed tests/test_zero3.py:94-147, on device buffers."""
    torch.manual_seed(0)
    params = [nn.Parameter(torch.randn(7, 5, device=DEV)), nn.Parameter(torch.randn(3, device=DEV))]
    originals = [p.data.clone() for p in params]
    g = FlatParamGroup(params, rank=1, world_size=2, zero_stage=3, device=torch.device(DEV))
    g.copy_model_to_flat()
    g.partition_params()
    assert g.data.numel() == g.numel_padded // 2 and g.shard_start == g.numel_padded // 2
    assert sum(p.numel() for p in params) == g.numel_shard()
    assert all(p.data.dim() == 1 for p in params)
    full = torch.cat([o.reshape(-1) for o in originals] + [torch.zeros(g.numel_padded - g.numel, device=DEV)])
    g.materialize_params()
    g.copy_flat_to_model(full)
    for p, o in zip(params, originals):
        assert torch.equal(p.data, o)
    g.dematerialize_params()
    g.copy_flat_to_model()
    off = 0
    for p, o in zip(params, originals):
        n = o.numel()
        lo, hi = max(off, g.shard_start), min(off + n, g.shard_end)
        assert p.data.numel() == max(0, hi - lo)
        if hi > lo:
            assert torch.equal(p.data, o.reshape(-1)[lo - off:hi - off])
        off += n
    g.materialize_params()
    g.copy_flat_to_model(full)
    for p, o in zip(params, originals):
        assert torch.equal(p.data, o)


@pytest.mark.parametrize("dtype,stage", [("fp16", 2), ("bf16", 1), ("fp32", 3), ("fp16", 3)])
def test_materialized_flat_grad_mode_is_bitwise_identical(dtype, stage):
    x, y = make_batch(3, GAS, MICRO)
    res = []
    for materialize in (False, True):
        model = build_model()
        engine = ms.initialize(model=model, model_parameters=list(model.parameters()),
                               config=config(dtype=dtype, stage=stage, materialize=materialize,
                                             lr=1e-2))
        train(engine, x, y, 3, GAS)
        res.append((engine.flat_groups[0].data.clone(),
                     engine.optimizer.state[0]["exp_avg_sq"].clone(), engine.grad_norm))
        g = engine.flat_groups[0]
        if stage < 3:
            assert not g.grad.any()          # zero after the boundary, as in the reference
        else:
            assert g.grad is None
    assert torch.equal(res[0][0], res[1][0]) and torch.equal(res[0][1], res[1][1])
    assert res[0][2] == res[1][2]


def test_has_overflow_on_device_buffers():
    assert not has_overflow(torch.zeros(4, device=DEV))
    assert has_overflow(torch.tensor([1.0, float("inf")], device=DEV))
    assert has_overflow(torch.tensor([float("nan")], device=DEV, dtype=torch.float16))
    assert has_overflow(torch.zeros(2, device=DEV), torch.tensor([float("-inf")], device=DEV,
                                                                 dtype=torch.bfloat16))
    big = torch.zeros(3_000_001, device=DEV)
    big[2_999_999] = float("nan")
    assert has_overflow(big) and not has_overflow(big[:2_999_999])


def test_two_param_groups_with_own_hyperparameters():
    model = build_model()
    groups = [{"params": list(model.net[0].parameters()), "lr": 3e-3, "weight_decay": 0.0},
              {"params": [p for m in list(model.net)[1:] for p in m.parameters()]}]
    engine = ms.initialize(model=model, model_parameters=groups, config=config(lr=1e-3))
    assert len(engine.flat_groups) == 2
    assert [g["lr"] for g in engine.optimizer.param_groups] == [3e-3, 1e-3]
    x, y = make_batch(2, GAS, MICRO)
    train(engine, x, y, 2, GAS)
    assert engine.global_steps == 2
    assert all(st["step"] == 2 for st in engine.optimizer.state)


def test_boundaries_on_alternating_streams_match_one_stream():
    """step() returns before K3 finishes; a boundary issued on another
    stream must still see the previous one complete (Workspace.enter)."""
    x, y = make_batch(4, GAS, MICRO)
    results = []
    for alternate in (False, True):
        model = build_model()
        engine = ms.initialize(model=model, model_parameters=list(model.parameters()),
                               config=config(dtype="fp16", lr=1e-2))
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        for s in range(4):
            for m in range(GAS):
                engine.backward(mse(engine(x[s, m]), y[s, m]))
            if alternate:
                st = streams[s % 2]
                st.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(st):
                    assert engine.step() is True
                torch.cuda.current_stream().wait_stream(st)
            else:
                assert engine.step() is True
        torch.cuda.synchronize()
        results.append((engine.flat_groups[0].data.clone(), engine.optimizer.state[0]["exp_avg_sq"].clone(),
                        engine.grad_norm))
    assert torch.equal(results[0][0], results[1][0]) and torch.equal(results[0][1], results[1][1])
    assert results[0][2] == results[1][2]


@pytest.mark.parametrize("materialize", [False, True])
def test_gradients_from_another_stream_outlive_the_boundary_kernels(materialize):
    """Gradients allocated on a producer stream, step() on a consumer
    stream, then, with no wait, the producer allocates and fills tensors of
    the same size: the caching allocator must not hand the gradients'
    memory to the producer while K1 / K3 on the consumer still read it.
    The run must equal the same steps taken on one stream."""
    n = 1 << 25
    cfg = {"train_micro_batch_size_per_gpu": 1, "gradient_accumulation_steps": 1,
           "gradient_clipping": 1.0, "dtype": "fp16",
           "fp16": {"enabled": True, "loss_scale": 0, "initial_scale_power": 16},
           "optimizer": {"type": "AdamW", "params": {"lr": 1e-3, "weight_decay": 0.01}},
           "hip_boundary": {"materialize_flat_grad": materialize}}
    gen = torch.Generator().manual_seed(11)
    host_grads = [(torch.randn(n, generator=gen) * 1e-3 * 2.0 ** 16).half() for _ in range(3)]
    init = torch.randn(n, generator=gen) * 0.02
    results = []
    for split in (False, True):
        p = nn.Parameter(init.clone().to(DEV))
        engine = ms.initialize(model=nn.ParameterList([p]), model_parameters=[p], config=cfg)
        producer, consumer = torch.cuda.Stream(), torch.cuda.Stream()
        for hg in host_grads:
            with torch.cuda.stream(producer):
                p.grad = hg.to(DEV)                     # allocated on the producer stream
            consumer.wait_stream(producer)
            with torch.cuda.stream(consumer if split else producer):
                engine.micro_steps += 1
                assert engine.step() is True
            with torch.cuda.stream(producer):           # no wait on the consumer
                junk = torch.full((n,), float("nan"), dtype=torch.float16, device=DEV)
                del junk
        torch.cuda.synchronize()
        results.append((engine.flat_groups[0].data.clone(),
                        engine.optimizer.state[0]["exp_avg_sq"].clone(), engine.grad_norm))
    assert torch.equal(results[0][0], results[1][0]) and torch.equal(results[0][1], results[1][1])
    assert results[0][2] == results[1][2]
    assert torch.isfinite(results[1][0]).all()


def test_thousands_of_tiny_tensors_against_the_oracle():
    """3000 parameters of 1..300 elements (segment tables of thousands of
    rows, most tiles straddling segment edges), fp16, ZeRO-2, clip: every
    boundary against the oracle started from the GPU's own state."""
    from oracle import boundary as ob
    from tests.helpers import clip_override, master_step_within_ulps, step_hyper

    rng = np.random.default_rng(5)
    sizes = rng.integers(1, 301, size=3000)
    gen = torch.Generator().manual_seed(9)
    init = [torch.randn(int(n), generator=gen) * 0.02 for n in sizes]
    params = [nn.Parameter(t.clone().to(DEV)) for t in init]
    module = nn.ParameterList(params)
    engine = ms.initialize(model=module, model_parameters=list(module),
                           config=config(dtype="fp16", stage=2, lr=1e-3, power=12, gas=1))
    ref_params = [nn.Parameter(t.clone()) for t in init]
    ref = ob.Engine([ref_params], [{"lr": 1e-3, "betas": (0.9, 0.999), "eps": 1e-8,
                                    "weight_decay": 0.01}], dtype="fp16", zero_stage=2, clip=1.0,
                    initial_scale_power=12, loss_scale_window=100,
                    scheduler_params={"warmup_max_lr": 1e-3})
    g = engine.flat_groups[0]
    assert len(g.boundary_table(0, g.numel_padded, g.grad_pointers()[0], None)) >= 3000
    for step in range(3):
        grads = [(torch.randn(int(n), generator=gen) * 1e-2 * 2.0 ** 12).half() for n in sizes]
        before = g.data.detach().cpu()
        st = engine.optimizer.state[0]
        ref.load_state([before], [st["exp_avg"].cpu()], [st["exp_avg_sq"].cpu()], [st["step"]],
                       (engine.loss_scaler.scale, engine.loss_scaler.good_steps,
                        engine.loss_scaler.skipped_steps),
                       engine.lr_scheduler.last_epoch, [pg["lr"] for pg in engine.optimizer.param_groups])
        for p, rp, gr in zip(params, ref_params, grads):
            p.grad = gr.to(DEV)
            rp.grad = gr.clone()
        engine.micro_steps += 1
        ref.micro_steps += 1
        hp = step_hyper(engine)
        assert engine.step() is True and ref.step(clip_override=clip_override(engine)) is True
        assert abs(engine.grad_norm - ref.grad_norm) <= 1e-5 * ref.grad_norm
        ok, worst, nsq = master_step_within_ulps(before.numpy(), g.data.cpu().numpy(),
                                                 ref.groups[0].data.numpy(), st["exp_avg"].cpu().numpy(),
                                                 st["exp_avg_sq"].cpu().numpy(), **hp)
        assert ok, (step, worst, nsq)
        assert torch.equal(st["exp_avg"].cpu(), ref.state[0]["exp_avg"])
        assert torch.equal(st["exp_avg_sq"].cpu(), ref.state[0]["exp_avg_sq"])
        master = g.data.cpu()
        for (off, p), n in zip(g._offsets, g._numels):
            assert torch.equal(p.detach().cpu().view(torch.int16),
                               master[off:off + n].to(torch.float16).view(torch.int16))


@pytest.mark.parametrize("stage", [0, 3])
def test_zero_size_parameter_in_the_list(stage):
    """An empty parameter among the others changes nothing for them."""
    from oracle import boundary as ob

    shapes = [(5, 3), (0, 4), (7,), (0,), (33,)]
    gen = torch.Generator().manual_seed(2)
    init = [torch.randn(*s, generator=gen) * 0.02 for s in shapes]
    params = [nn.Parameter(t.clone().to(DEV)) for t in init]
    module = nn.ParameterList(params)
    engine = ms.initialize(model=module, model_parameters=list(module),
                           config=config(dtype="fp16", stage=stage, gas=1, lr=1e-2))
    ref_params = [nn.Parameter(t.clone()) for t in init]
    ref = ob.Engine([ref_params], [{"lr": 1e-2, "betas": (0.9, 0.999), "eps": 1e-8,
                                    "weight_decay": 0.01}], dtype="fp16", zero_stage=stage, clip=1.0,
                    initial_scale_power=8, loss_scale_window=100,
                    scheduler_params={"warmup_max_lr": 1e-2})
    for step in range(3):
        if stage >= 3:
            engine.optimizer.gather_parameters()
            ref.gather_parameters()
        grads = [(torch.randn(*s, generator=gen) * 256.0 * 1e-2).half() for s in shapes]
        for p, rp, g in zip(params, ref_params, grads):
            p.grad = g.to(DEV)
            rp.grad = g.clone()
        engine.micro_steps += 1
        ref.micro_steps += 1
        assert engine.step() is True and ref.step() is True
        assert abs(engine.grad_norm - ref.grad_norm) <= 1e-5 * ref.grad_norm
        np.testing.assert_allclose(engine.flat_groups[0].data.cpu().numpy(), ref.groups[0].data.numpy(),
                                   rtol=1e-6, atol=1e-7)
    if stage >= 3:
        engine.optimizer.gather_parameters()
    assert [tuple(p.shape) for p in params] == shapes


def test_state_arena_windows():
    """With a window the buffers lie in one allocation of three windows:
    array j of every group at window j, the groups back to back at the same
    offsets (2 MiB slots), zeroed.  The arena is carved through torch's
    caching allocator: the buffers hold only their slots, and the windows'
    unused part is free memory of the allocator that later tensors are
    served from.  A column larger than a window, or no window, gives
    separate allocations."""
    from minispeed_amd.flat import place_state

    dev = torch.device(DEV)
    mib = 1 << 20
    win = 512 * mib
    sizes = [[1000, 700, 700], [mib // 4 + 3, mib // 4 + 3, 5]]
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    def large_reserved():
        return torch.cuda.memory_stats(dev)["reserved_bytes.large_pool.current"]

    before = torch.cuda.memory_allocated(dev)
    reserved = large_reserved()
    bufs, placement = place_state(sizes, dev, win)
    torch.cuda.synchronize()
    assert [[b.numel() for b in row] for row in bufs] == sizes
    flat_bufs = [b for row in bufs for b in row]
    assert all(b.dtype == torch.float32 and b.is_contiguous() and int(b.count_nonzero()) == 0
               for b in flat_bufs)
    base = bufs[0][0].data_ptr()
    for j in range(3):
        assert bufs[0][j].data_ptr() - base == j * win
        assert bufs[1][j].data_ptr() - base == j * win + 2 * mib     # after group 0's 2 MiB slot
    assert placement.window == win and placement.arena_bytes == 3 * win
    assert placement.held_bytes == 6 * 2 * mib
    assert placement.returned_bytes == 3 * win - 12 * mib
    # the state holds its slots only; the arena is one new segment of 3 windows
    assert torch.cuda.memory_allocated(dev) - before == 12 * mib
    assert large_reserved() - reserved == 3 * win
    # tensors allocated afterwards are served from the windows' gaps: no new segment
    later = [torch.empty(400 * mib, dtype=torch.uint8, device=dev) for _ in range(3)]
    assert all(base <= t.data_ptr() and t.data_ptr() + t.numel() <= base + 3 * win for t in later)
    assert large_reserved() - reserved == 3 * win
    for t in later:
        t.fill_(0xFF)
    torch.cuda.synchronize()
    assert all(int(b.count_nonzero()) == 0 for b in flat_bufs)
    bufs[1][1].fill_(1.0)
    assert all(int(b.count_nonzero()) == 0 for b in flat_bufs if b is not bufs[1][1])
    del later
    big, big_place = place_state([[300 * mib, 10, 10]], dev, win)    # 1200 MiB > 512 MiB window
    assert len({b.untyped_storage().data_ptr() for b in big[0]}) == 3 and big_place.window == 0
    plain, plain_place = place_state([[1000, 1000, 1000]], dev, 0)
    assert len({b.untyped_storage().data_ptr() for b in plain[0]}) == 3
    assert plain_place.arena_bytes == 0 and plain_place.returned_bytes == 0


_ARENA_NO_SPLIT = r"""
import json, torch
from minispeed_amd.flat import place_state
dev = torch.device("cuda", 0)
mib = 1 << 20
torch.zeros(1, device=dev)
before = torch.cuda.memory_reserved(dev)
bufs, where = place_state([[100 * mib, 100 * mib, 100 * mib]], dev, 512 * mib)
grown = torch.cuda.memory_reserved(dev) - before
ok = all(int(b.count_nonzero()) == 0 and b.numel() == 100 * mib for b in bufs[0])
base = bufs[0][0].data_ptr()
offs = [b.data_ptr() - base for b in bufs[0]]
print(json.dumps({"arena": where.arena_bytes, "held": where.held_bytes,
                  "returned": where.returned_bytes, "grown": grown, "zero": ok, "offs": offs}))
"""


def test_state_arena_when_the_allocator_will_not_split_it():
    """With ``max_split_size_mb`` below the arena's size torch's caching
    allocator never splits the arena's block, so the state slots cannot be
    carved out of it: place_state stops at the first request that would
    take a new segment and keeps the whole arena as one tensor (the windows
    still 512 MiB apart), without allocating more.  Runs in a child process:
    the allocator setting is read when the process first allocates."""
    import json
    import os
    import subprocess
    import sys

    env = dict(os.environ)
    env["PYTORCH_HIP_ALLOC_CONF"] = "max_split_size_mb:1024"
    env.pop("PYTORCH_CUDA_ALLOC_CONF", None)
    env.pop("PYTORCH_ALLOC_CONF", None)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    out = subprocess.run([sys.executable, "-c", _ARENA_NO_SPLIT], cwd=root, env=env,
                         capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr[-2000:]
    res = json.loads(out.stdout.strip().splitlines()[-1])
    mib = 1 << 20
    assert res["arena"] == 3 * 512 * mib and res["held"] == res["arena"] and res["returned"] == 0
    assert res["offs"] == [0, 512 * mib, 1024 * mib] and res["zero"]
    # the arena, plus the one segment the first carving request (a 400 MiB
    # slot) took before the carve gave up
    assert res["grown"] <= 3 * 512 * mib + 400 * mib, res["grown"]


def test_two_groups_share_one_arena():
    module = nn.Sequential(nn.Linear(64, 32), nn.Linear(32, 8)).to(DEV)
    decay = [p for n, p in module.named_parameters() if n.endswith("weight")]
    no_decay = [p for n, p in module.named_parameters() if n.endswith("bias")]
    cfg = config(dtype="bf16", stage=1, gas=1)
    cfg["hip_boundary"] = {"state_spacing_gib": 0.01}
    engine = ms.initialize(model=module, model_parameters=[{"params": decay},
                                                           {"params": no_decay, "weight_decay": 0.0}],
                           config=cfg)
    g0, g1 = engine.flat_groups
    st0, st1 = engine.optimizer.state
    win = st0["exp_avg"].data_ptr() - g0.data.data_ptr()
    assert win == engine.state_placement.window > 0
    assert st0["exp_avg_sq"].data_ptr() - st0["exp_avg"].data_ptr() == win
    assert st1["exp_avg"].data_ptr() - g1.data.data_ptr() == win
    assert g1.data.data_ptr() - g0.data.data_ptr() == 2 << 20
    assert g0.state_placement is g1.state_placement is engine.state_placement


@pytest.mark.parametrize("stage", [1, 3])
def test_state_spacing_changes_no_result(stage):
    """The same steps with the masters and moments in a spaced arena and in
    separate allocations give bitwise the same masters, moments and model."""
    runs = []
    for spacing in (0, 0.01):
        torch.manual_seed(0)
        module = nn.Sequential(nn.Linear(96, 64), nn.GELU(), nn.Linear(64, 8)).to(DEV)
        cfg = config(dtype="fp16", stage=stage, gas=1)
        cfg["hip_boundary"] = {"state_spacing_gib": spacing}
        engine = ms.initialize(model=module, model_parameters=list(module.parameters()), config=cfg)
        gen = torch.Generator().manual_seed(1)
        for _ in range(3):
            if stage >= 3:
                engine.optimizer.gather_parameters()
            x = torch.randn(16, 96, generator=gen).to(DEV).half()
            loss = engine(x).float().pow(2).mean()
            engine.backward(loss)
            engine.step()
        if stage >= 3:
            engine.optimizer.gather_parameters()
        st = engine.optimizer.state[0]
        runs.append([engine.flat_groups[0].data.clone(), st["exp_avg"].clone(), st["exp_avg_sq"].clone()]
                    + [p.detach().clone() for p in module.parameters()])
    for a, b in zip(*runs):
        assert torch.equal(a.view(torch.int8), b.view(torch.int8))


def test_engine_takes_the_moments_allocated_with_the_masters():
    module = nn.Linear(64, 32).to(DEV)
    engine = ms.initialize(model=module, model_parameters=list(module.parameters()),
                           config=config(dtype="bf16", stage=1, gas=1))
    g = engine.flat_groups[0]
    assert g.take_moment_buffers() is None            # handed to the optimizer
    st = engine.optimizer.state[0]
    assert st["exp_avg"].numel() == st["exp_avg_sq"].numel() == g.numel_shard()


def test_owned_range_table_uses_the_gradient_element_size():
    """A table over one rank's range starts rows mid-parameter; the gradient
    address of such a row advances by the gradient's element size (4 for the
    fp32 sums of contiguous gradients, 2 for fp16 parameters' own grads)."""
    params = [nn.Parameter(torch.zeros(n, dtype=torch.float16, device=DEV)) for n in (10, 7, 13)]
    g = FlatParamGroup(params, rank=1, world_size=2, zero_stage=1, device=torch.device(DEV))
    lo, hi = g.own_range                                   # [15, 30): starts inside param 1
    assert (lo, hi) == (15, 30)
    gptrs = [1 << 20, 2 << 20, 3 << 20]
    for esize in (4, 2, None):
        table = g.boundary_table(lo, hi, gptrs, None, esize)
        step = esize or 2
        rows = {int(b): (int(n), int(gp)) for b, n, gp, _ in table}
        assert rows[15] == (2, (2 << 20) + (15 - 10) * step)     # param 1, elements 5..6
        assert rows[17] == (13, 3 << 20)                          # param 2 from its start
