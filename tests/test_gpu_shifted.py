"""Segments off the alignment of the flat space.

The flat layout packs tensors back to back (flat.py:FlatParamGroup, as
minispeed's), so one tensor of a size that is not a multiple of 8 puts every
later gradient and model copy off the 16-byte units of K1's tiles and the
quads of K3's; gradient and model views can also start at any element of
their storage.  The kernels keep those tiles on vector paths (K1: the walk
of a tile's head, tail and units, its ends loaded with the first units,
rounds predicated; when writing the flat gradient, the tile split over
the block's four waves with its head and tail staged in LDS; K3 /
K4 / K5: quads of any alignment).  Checked here:

* K1's pure flatten (the initial master copy) of shifted tensors of whole
  tiles, bit for bit;
* K1 for every head length and dtype: the flat gradient bit for bit against
  the widened, scaled gradients, every tile flag exactly, tile sums within
  1e-12 of the exact sum of squares, and the statistics bit for bit the same
  with and without the flat output;
* K3 over a packed layout whose gradients and model copies have every quad
  kind, bit for bit against K3 over the same tensors laid out on whole
  tiles (the per-element arithmetic is the same, so every master, moment
  and model element must be too);
* K4's model copies of every kind against torch's casts, K5's gradient at
  2 mod 4 bytes against the fp32 sum;
* an engine on a shifted GPT-like list against the oracle, step by step;
  with the flat gradient materialised against the fused mode, bit for bit;
  and ZeRO-3 (parameters gathered as views at odd offsets of one buffer)
  against stage 0 bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

import minispeed_amd as ms
from minispeed_amd import _native
from oracle import boundary as ob
from oracle import recipe
from tests.helpers import (DEV, Table, adamw_params, bits, clip_override, k1, k3, k4, layout_for,
                           master_step_within_ulps, scalars_device, step_hyper, store)

pytestmark = pytest.mark.gpu

F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32
TILE = _native.SCAN_TILE


def _views(sizes, dtype, offsets, fill=0.0):
    """One pool per tensor list: tensor i a view starting offsets[i]
    elements past a 16-byte boundary of the pool."""
    views = []
    pool = torch.full((sum(sizes) + 16 * len(sizes) + 16,), fill, dtype=dtype, device=DEV)
    per16 = 16 // pool.element_size()
    pos = 0
    for k, off in zip(sizes, offsets):
        pos = -(-pos // per16) * per16 + off
        views.append(pool[pos:pos + k])
        pos += k
    return pool, views


def _assert_outside_untouched(pool, views, fill):
    """Every element of the pool that no view covers still holds ``fill``:
    the kernels wrote nothing outside the tensors."""
    covered = torch.zeros(pool.numel(), dtype=torch.bool)
    base = pool.data_ptr()
    for v in views:
        i = (v.data_ptr() - base) // pool.element_size()
        covered[i:i + v.numel()] = True
    rest = pool.cpu()[~covered]
    assert torch.all(rest == fill), "a kernel wrote outside the tensors"


@pytest.mark.parametrize("dtype", [F16, BF16, F32])
@pytest.mark.parametrize("head", range(8))
def test_k1_every_head_length(dtype, head):
    """A first tensor of `head` elements shifts the rest; a missing gradient
    spans whole tiles; the owned range cuts tiles; the flat output is
    written with and without the statistics."""
    sizes = [head, 5 * TILE + 3, 3 * TILE, 77, 4 * TILE + 1, 2 * TILE + 5]
    sizes = [s for s in sizes if s]
    missing = {len(sizes) - 3}                # the 4-tile + 1 tensor
    gen = torch.Generator().manual_seed(11 + head)
    host = [(torch.randn(k, generator=gen) * 1e-2).to(dtype) for k in sizes]
    if head % 3 == 1:                         # an inf in a shifted tile
        host[1][TILE + 9] = float("inf")
    _, views = _views(sizes, dtype, [0] * len(sizes))
    for v, h in zip(views, host):
        v.copy_(h.to(DEV))
    lay = layout_for(sizes)
    n = lay.numel_padded
    gst = [None if i in missing else store(v, off)
           for i, (v, off) in enumerate(zip(views, lay.offsets))]
    tab = Table(lay, 0, n, gst, [None] * len(sizes))
    full = torch.zeros(n)
    for i, (h, off) in enumerate(zip(host, lay.offsets)):
        if i not in missing:
            full[off:off + h.numel()] = h.float()
    scale = 2.0 ** 3 if dtype == F16 else 1.0
    want = full / scale if scale != 1.0 else full
    for lo, hi in ((0, n), (TILE + 3, n - 2 * TILE - 1)):
        flat = torch.full((n,), float("nan"), device=DEV)
        with_flat = k1(tab, dtype, 0, n, lo, hi, scale=scale, flat=flat, tiles=True)
        without = k1(tab, dtype, 0, n, lo, hi, scale=scale, tiles=True)
        for a, b in zip(with_flat, without):
            np.testing.assert_array_equal(a.view(np.uint8), b.view(np.uint8))
        np.testing.assert_array_equal(bits(flat), bits(want))
        _, _, ts, tf = without
        owned = want.numpy().astype(np.float64)
        owned[:lo] = 0.0
        owned[hi:] = 0.0
        bad = ~np.isfinite(full.numpy())
        for t in range(ts.size):
            a, b = t * TILE, min((t + 1) * TILE, n)
            assert bool(tf[t]) == bool(bad[a:b].any()), t
            if not bad[a:b].any():
                exact = recipe.sumsq_f64(owned[a:b].astype(np.float32))
                assert abs(ts[t] - exact) <= 1e-12 * exact, t


@pytest.mark.parametrize("dtype", [F16, BF16, F32])
@pytest.mark.parametrize("head", [1, 3, 5, 6])
def test_k1_flatten_only_of_shifted_tensors(dtype, head):
    """The pure ragged flatten (no statistics, as copy_model_to_flat) over
    tensors of whole tiles behind a `head`-element one, over the whole flat
    space and over a sub-range that starts off the tile grid: every output
    element is the widened source, bit for bit, and nothing past the range
    is written."""
    sizes = [head, 5 * TILE + 3, 3 * TILE, 77, 4 * TILE + 1, 2 * TILE]
    gen = torch.Generator().manual_seed(31 + head)
    host = [torch.randn(k, generator=gen).to(dtype) for k in sizes]
    _, views = _views(sizes, dtype, [0] * len(sizes))
    for v, h in zip(views, host):
        v.copy_(h.to(DEV))
    lay = layout_for(sizes)
    n = lay.numel_padded
    full = torch.zeros(n)
    for h, off in zip(host, lay.offsets):
        full[off:off + h.numel()] = h.float()
    gst = [store(v, off) for v, off in zip(views, lay.offsets)]
    lib = _native.load()
    for lo, hi in ((0, n), (TILE + 5, n - TILE - 3)):
        tab = Table(lay, lo, hi, gst, [None] * len(sizes))
        flat = torch.full((hi - lo + 64,), float("nan"), device=DEV)
        _native.check(lib.ms_grad_stats(tab.ptr, tab.nseg, _native.ms_dtype(dtype), lo, hi, lo, hi,
                                        0, 1.0, flat.data_ptr(), None, None, 0, None, None, 0,
                                        _native.stream_handle(torch.device(DEV))), "flatten")
        torch.cuda.synchronize()
        got = flat.cpu()
        np.testing.assert_array_equal(bits(got[:hi - lo]), bits(full[lo:hi]))
        assert torch.isnan(got[hi - lo:]).all(), "wrote past the range"


COMBOS = [(F16, F16), (BF16, BF16), (F32, F32), (F16, F32), (F32, BF16), (BF16, F16)]


@pytest.mark.parametrize("gdtype,mdtype", COMBOS)
@pytest.mark.parametrize("flat_grad", [False, True], ids=["ragged", "flat_grad"])
def test_k3_quads_of_every_kind_match_the_aligned_layout(gdtype, mdtype, flat_grad):
    sizes = [3, 9 * 512 + 1, 2, 5 * 512 + 7, 6 * 512, 1, 4 * 512 + 2]
    rng = np.random.default_rng(3)
    gen = torch.Generator().manual_seed(5)
    host_g = [(torch.randn(k, generator=gen) * 1e-2).to(gdtype) for k in sizes]
    p0 = [rng.normal(0, 0.02, k).astype(np.float32) for k in sizes]
    m0 = [rng.normal(0, 1e-3, k).astype(np.float32) for k in sizes]
    v0 = [(rng.random(k) * 1e-6).astype(np.float32) for k in sizes]
    hp = adamw_params(1e-3, (0.9, 0.999), 1e-8, 0.01, 5)
    sc = scalars_device(clip_applied=1, coef=0.61)

    def run(layout_sizes, index, g_offsets, m_offsets):
        """K3 over a layout of `layout_sizes` in which tensor i sits at
        position index[i] (the others are padding: no gradient, no model)."""
        lay = layout_for(layout_sizes)
        n = lay.numel_padded
        _, gviews = _views(sizes, gdtype, g_offsets)
        mpool, mviews = _views(sizes, mdtype, m_offsets, fill=7.0)
        for v, h in zip(gviews, host_g):
            v.copy_(h.to(DEV))
        gst = [None] * len(layout_sizes)
        mst = [None] * len(layout_sizes)
        p, m, v = (np.zeros(n, np.float32) for _ in range(3))
        fg = np.zeros(n, np.float32)
        for i, j in enumerate(index):
            off = lay.offsets[j]
            gst[j] = store(gviews[i], off)
            mst[j] = store(mviews[i], off)
            p[off:off + sizes[i]] = p0[i]
            m[off:off + sizes[i]] = m0[i]
            v[off:off + sizes[i]] = v0[i]
            fg[off:off + sizes[i]] = host_g[i].float().numpy()
        dp, dm, dv = (torch.from_numpy(x).to(DEV) for x in (p, m, v))
        if flat_grad:
            tab = Table(lay, 0, n, [None] * len(layout_sizes), mst)
            k3(tab, gdtype, mdtype, 0, n, dp, dm, dv, hp, sc,
               flat_grad=torch.from_numpy(fg).to(DEV))
        else:
            tab = Table(lay, 0, n, gst, mst)
            k3(tab, gdtype, mdtype, 0, n, dp, dm, dv, hp, sc)
        out = []
        for i, j in enumerate(index):
            off = lay.offsets[j]
            out.append([x[off:off + sizes[i]].cpu() for x in (dp, dm, dv)] + [mviews[i].cpu()])
        _assert_outside_untouched(mpool, mviews, 7.0)
        return out

    # packed, views at every element offset of 16 bytes
    per16 = 16 // torch.empty(0, dtype=gdtype).element_size()
    shifted = run(sizes, list(range(len(sizes))), [i % per16 for i in range(len(sizes))],
                  [(3 * i + 1) % (16 // torch.empty(0, dtype=mdtype).element_size())
                   for i in range(len(sizes))])
    # every tensor on whole 512-element tiles, storage 16-byte aligned
    padded, index = [], []
    for k in sizes:
        index.append(len(padded))
        padded.append(k)
        pad = -k % 512
        if pad:
            padded.append(pad)
    aligned = run(padded, index, [0] * len(sizes), [0] * len(sizes))
    for i, (a, b) in enumerate(zip(shifted, aligned)):
        for name, x, y in zip(("master", "exp_avg", "exp_avg_sq", "model"), a, b):
            np.testing.assert_array_equal(bits(x), bits(y), err_msg=f"tensor {i} {name}")


@pytest.mark.parametrize("mdtype", [F16, BF16, F32])
@pytest.mark.parametrize("shift", [0, 1, 2, 3])
def test_k4_model_copies_of_every_kind(mdtype, shift):
    """Shifts 1 and 3 put every whole tile of a 2-byte model type at 2 mod 4
    bytes (the whole-word stores of the kind-2 path), 0 and 2 at kinds 0
    and 1."""
    sizes = [5, 4 * 1024 + 3, 1, 8 * 1024, 3 * 1024 + 2, 7]
    lay = layout_for(sizes)
    n = lay.numel_padded
    per16 = 16 // torch.empty(0, dtype=mdtype).element_size()
    pool, mviews = _views(sizes, mdtype, [(i * 3 + shift) % per16 for i in range(len(sizes))],
                          fill=9.0)
    flat = torch.randn(n, generator=torch.Generator().manual_seed(2)) * 3.0
    tab = Table(lay, 0, n, [None] * len(sizes),
                [store(v, off) for v, off in zip(mviews, lay.offsets)])
    k4(tab, mdtype, flat.to(DEV), 0, n)
    for v, off, k in zip(mviews, lay.offsets, sizes):
        np.testing.assert_array_equal(bits(v), bits(flat[off:off + k].to(mdtype)))
    _assert_outside_untouched(pool, mviews, 9.0)


@pytest.mark.parametrize("dtype", [F16, BF16])
@pytest.mark.parametrize("goff", [1, 3])
def test_k5_gradient_at_2_mod_4_bytes(dtype, goff):
    lib = _native.load()
    n = 100003
    gen = torch.Generator(device=DEV).manual_seed(goff)
    pool = torch.zeros(n + 16, dtype=dtype, device=DEV)
    src = pool[goff:goff + n]
    buf = torch.full((n + 9,), -3.0, device=DEV)
    stream = _native.stream_handle(torch.device(DEV))
    want = None
    for k in range(2):
        src.copy_(torch.randn(n, generator=gen, device=DEV).to(dtype))
        _native.check(lib.ms_accumulate_grad(buf.data_ptr() + 4, src.data_ptr(),
                                             _native.ms_dtype(dtype), n, 1 if k == 0 else 0,
                                             stream), "ms_accumulate_grad")
        want = ob.accumulate_fp32(want, src.cpu())
        np.testing.assert_array_equal(bits(buf[1:1 + n]), bits(want))
    assert buf[0].item() == -3.0 and torch.all(buf[1 + n:].cpu() == -3.0)
    assert torch.all(pool[:goff].cpu() == 0) and torch.all(pool[goff + n:].cpu() == 0)


@pytest.mark.parametrize("dtype,stage", [("fp16", 0), ("fp16", 1), ("bf16", 2)])
def test_engine_on_a_shifted_list_against_the_oracle(dtype, stage):
    """A 3-element tensor first, then GPT-like blocks: every later tensor off
    the flat space's alignment; three boundaries against the oracle."""
    sizes = [3, 96 * 64, 64, 3 * 64 * 64, 192, 4 * 64 * 64, 256, 5, 64 * 4 * 64, 64]
    tdt = {"fp16": torch.float16, "bf16": torch.bfloat16}[dtype]
    gen = torch.Generator().manual_seed(21)
    init = [torch.randn(n, generator=gen) * 0.02 for n in sizes]
    params = [nn.Parameter(t.clone().to(DEV)) for t in init]
    module = nn.ParameterList(params)
    cfg = {"train_micro_batch_size_per_gpu": 1, "gradient_accumulation_steps": 1,
           "gradient_clipping": 1.0, "dtype": dtype, "zero_optimization": {"stage": stage},
           "optimizer": {"type": "AdamW", "params": {"lr": 1e-3, "betas": [0.9, 0.999],
                                                      "eps": 1e-8, "weight_decay": 0.01}},
           "scheduler": {"type": "WarmupLR", "params": {"warmup_max_lr": 1e-3}},
           "steps_per_print": 1000}
    power = 12
    if dtype == "fp16":
        cfg["fp16"] = {"enabled": True, "loss_scale": 0, "initial_scale_power": power,
                       "loss_scale_window": 100}
    engine = ms.initialize(model=module, model_parameters=list(module), config=cfg)
    ref_params = [nn.Parameter(t.clone()) for t in init]
    ref = ob.Engine([ref_params], [{"lr": 1e-3, "betas": (0.9, 0.999), "eps": 1e-8,
                                    "weight_decay": 0.01}], dtype=dtype, zero_stage=stage,
                    clip=1.0, initial_scale_power=power, loss_scale_window=100,
                    scheduler_params={"warmup_max_lr": 1e-3})
    g = engine.flat_groups[0]
    mult = 2.0 ** power if dtype == "fp16" else 1.0
    for step in range(3):
        grads = [(torch.randn(n, generator=gen) * 1e-2 * mult).to(tdt) for n in sizes]
        before = g.data.detach().cpu()
        st = engine.optimizer.state[0]
        ref.load_state([before], [st["exp_avg"].cpu()], [st["exp_avg_sq"].cpu()], [st["step"]],
                       (engine.loss_scaler.scale, engine.loss_scaler.good_steps,
                        engine.loss_scaler.skipped_steps),
                       engine.lr_scheduler.last_epoch,
                       [pg["lr"] for pg in engine.optimizer.param_groups])
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
        np.testing.assert_array_equal(bits(p.detach().reshape(-1)), bits(master[off:off + n].to(tdt)))


@pytest.mark.parametrize("stage", [1, 2])
def test_materialized_flat_gradient_on_a_shifted_list_equals_fused(stage):
    """Tensors of whole tiles behind odd-sized ones (K1 writing the flat
    gradient splits those tiles over the block's waves, head and tail
    staged in LDS): three fp16 boundaries with the fp32 flat gradient
    materialised give bitwise the masters, moments, norms and model of the
    fused mode."""
    sizes = [3, 5 * TILE + 7, 64, 3 * TILE, 5, 4 * TILE + 1, 9 * TILE, 2]
    runs = []
    for materialize in (False, True):
        gen = torch.Generator().manual_seed(8)
        params = [nn.Parameter((torch.randn(n, generator=gen) * 0.02).to(DEV)) for n in sizes]
        module = nn.ParameterList(params)
        cfg = {"train_micro_batch_size_per_gpu": 1, "gradient_accumulation_steps": 1,
               "gradient_clipping": 0.5, "dtype": "fp16", "zero_optimization": {"stage": stage},
               "optimizer": {"type": "AdamW", "params": {"lr": 1e-3, "weight_decay": 0.01}},
               "fp16": {"enabled": True, "loss_scale": 0, "initial_scale_power": 10},
               "hip_boundary": {"materialize_flat_grad": materialize}, "steps_per_print": 1000}
        engine = ms.initialize(model=module, model_parameters=list(module), config=cfg)
        norms = []
        for _ in range(3):
            for p, n in zip(params, sizes):
                p.grad = (torch.randn(n, generator=gen) * 1e-2 * 2.0 ** 10).to(DEV).half()
            engine.micro_steps += 1
            assert engine.step() is True
            norms.append(engine.grad_norm)
        st = engine.optimizer.state[0]
        runs.append(([engine.flat_groups[0].data.clone(), st["exp_avg"].clone(),
                      st["exp_avg_sq"].clone()] + [p.detach().clone() for p in params], norms))
    (a, na), (b, nb) = runs
    assert na == nb and any(n > 0.5 for n in na)      # the clip ran
    for x, y in zip(a, b):
        assert torch.equal(x.view(torch.int8), y.view(torch.int8))


def test_zero3_on_a_shifted_list_equals_stage0():
    """ZeRO-3 gathers the parameters as views of one model-dtype buffer, here
    at odd element offsets (K3's and K4's model stores of every kind): the
    masters and the gathered parameters equal stage 0's bit for bit."""
    sizes = [3, 4099, 5, 8192, 77, 6000, 1]
    out = {}
    for stage in (0, 3):
        gen = torch.Generator().manual_seed(4)
        init = [torch.randn(n, generator=gen) * 0.02 for n in sizes]
        params = [nn.Parameter(t.to(DEV)) for t in init]
        module = nn.ParameterList(params)
        cfg = {"train_micro_batch_size_per_gpu": 1, "gradient_accumulation_steps": 1,
               "gradient_clipping": 1.0, "dtype": "fp16",
               "fp16": {"enabled": True, "loss_scale": 0, "initial_scale_power": 8},
               "optimizer": {"type": "AdamW", "params": {"lr": 1e-3, "weight_decay": 0.01}},
               "zero_optimization": {"stage": stage}, "steps_per_print": 1000}
        engine = ms.initialize(model=module, model_parameters=list(module), config=cfg)
        for _ in range(3):
            if stage == 3:
                engine.optimizer.gather_parameters()
            grads = [(torch.randn(n, generator=gen) * 1e-2 * 2.0 ** 8).half() for n in sizes]
            for p, gr in zip(params, grads):
                p.grad = gr.to(DEV)
            engine.micro_steps += 1
            assert engine.step() is True
        if stage == 3:
            engine.optimizer.gather_parameters()
        out[stage] = (engine.flat_groups[0].data.detach().cpu().clone(),
                      [p.detach().cpu().clone() for p in params])
    np.testing.assert_array_equal(bits(out[3][0]), bits(out[0][0]))
    for a, b in zip(out[3][1], out[0][1]):
        np.testing.assert_array_equal(bits(a), bits(b))
