"""Kernel parity through the C ABI: K1 (ragged scan), K2 (norm / clip /
skip / scale), K3 (fused AdamW + cast), K4 (cast) against the oracle.

Bars: flat grads, flags, casts, scaler decisions and the fused AdamW against
the kernel recipe (oracle.recipe) are bit-exact; the per-block fp64 sum of
squares agrees with an exact fp64 dot product to 1e-12 relative; AdamW
against the torch restatement (oracle.boundary) is bit-exact in exp_avg /
exp_avg_sq and within 2 fp32 ulp of max(|p_old|, |p_new|) in the master,
the only difference being torch's CPU sqrt.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch
from torch import nn

from minispeed_amd import _native
from oracle import boundary as ob
from oracle import recipe
from tests.helpers import (DEV, HALF_SPECIALS, Table, adamw_params, bits, k1, k2, k3, k4,
                           layout_for, master_step_within_ulps, ragged_grads, scalars_device,
                           set_bits, store, stream)

pytestmark = pytest.mark.gpu

F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32
RAGGED = [(7, 5), (3,), (3 * 2048,), (1,), (4099,), (64, 65), (10000,)]
ALIGNED = [(4096, 8), (8,), (5 * 2048,), (2048, 24)]


def _oracle_flat(shapes, grads, scale):
    dtype = next(g.dtype for g in grads if g is not None)
    params = [nn.Parameter(torch.zeros(*s, dtype=dtype)) for s in shapes]
    g = ob.Group(params)
    for p, gr in zip(params, grads):
        p.grad = None if gr is None else gr.clone()
    g.flatten_grads()
    flag = ob.has_overflow(g.grad)
    g.unscale_grads(scale)
    return g.grad, flag


def _device(grads):
    return [None if g is None else g.to(DEV) for g in grads]


def _grad_table(shapes, dgrads, world=1, rank=0, stage=0, lo=None, hi=None):
    lay = layout_for([int(np.prod(s)) for s in shapes], world, rank, stage)
    lo = 0 if lo is None else lo
    hi = lay.numel_padded if hi is None else hi
    gs = [store(g, off) for g, off in zip(dgrads, lay.offsets)]
    return lay, Table(lay, lo, hi, gs, [None] * len(shapes))


@pytest.mark.parametrize("dtype", [F16, BF16, F32])
@pytest.mark.parametrize("scale", [1.0, 65536.0, 1000.0])
@pytest.mark.parametrize("shapes", [RAGGED, ALIGNED], ids=["ragged", "aligned"])
def test_k1_flatten_unscale_and_sumsq(dtype, scale, shapes):
    grads = ragged_grads(shapes, dtype, 1e-3, seed=11, scale=scale if dtype == F16 else 1.0)
    grads[1] = None                                   # a parameter without gradient
    dg = _device(grads)
    lay, tab = _grad_table(shapes, dg)
    n = lay.numel_padded
    flat = torch.full((n,), float("nan"), device=DEV)
    psum, pflag = k1(tab, dtype, 0, n, 0, n, scale=scale, flat=flat)
    want, flag = _oracle_flat(shapes, grads, scale)
    assert not flag and not pflag.any()
    np.testing.assert_array_equal(bits(flat), bits(want))
    exact = recipe.sumsq_f64(want.numpy())
    assert abs(psum.sum() - exact) <= 1e-12 * exact


@pytest.mark.parametrize("dtype", [F16, BF16, F32])
def test_k1_flag_every_special_encoding(dtype):
    shapes = RAGGED
    specials = HALF_SPECIALS[dtype]
    for k, pattern in enumerate(specials):
        grads = ragged_grads(shapes, dtype, 1e-3, seed=20 + k)
        # put the special in a different parameter / position each time
        pi = [0, 2, 4, 5, 6, 3, 2, 6, 0][k]
        idx = [3, 2047, 4098, 4159, 9999, 0, 5000, 1, 34][k]
        set_bits(grads[pi], idx, pattern)
        dg = _device(grads)
        lay, tab = _grad_table(shapes, dg)
        n = lay.numel_padded
        psum, pflag = k1(tab, dtype, 0, n, 0, n)
        _, want = _oracle_flat(shapes, grads, 1.0)
        assert bool(pflag.any()) == want == (k < 5), (hex(pattern), pi, idx)
        s = k2(psum, pflag)
        assert bool(s.overflow) == want


def test_k1_partials_are_deterministic():
    shapes = ALIGNED + RAGGED
    grads = _device(ragged_grads(shapes, BF16, 1e-2, seed=3))
    lay, tab = _grad_table(shapes, grads)
    n = lay.numel_padded
    a = k1(tab, BF16, 0, n, 0, n)[0]
    b = k1(tab, BF16, 0, n, 0, n)[0]
    np.testing.assert_array_equal(a.view(np.int64), b.view(np.int64))


@pytest.mark.parametrize("dtype", [F16, BF16, F32])
@pytest.mark.parametrize("layout", ["ragged", "aligned", "misaligned", "shard"])
def test_k1_tile_statistics_do_not_depend_on_the_flat_output(dtype, layout):
    """Writing the flat gradient changes no statistics bit (the piece paths
    depend on the gradient storage alone), and tile t's fp64 sum is the
    exact sum of squares of its owned elements [t*2048, (t+1)*2048) to
    1e-12: the tile boundaries sit where the header says."""
    shapes = ALIGNED + RAGGED if layout != "aligned" else ALIGNED
    grads = ragged_grads(shapes, dtype, 1e-3, seed=41)
    dg = _device(grads)
    if layout == "misaligned":
        # 2-byte (fp16/bf16) or 4-byte (fp32) aligned storage: per-element path
        for k in (0, 3):
            base = torch.zeros(dg[k].numel() + 1, dtype=dtype, device=DEV)
            base[1:].copy_(dg[k].reshape(-1))
            dg[k] = base[1:].view(dg[k].shape)
            assert dg[k].data_ptr() % 16 != 0
    world, rank, stage = (3, 1, 2) if layout == "shard" else (1, 0, 0)
    lay, tab = _grad_table(shapes, dg, world, rank, stage)
    n = lay.numel_padded
    lo, hi = (lay.shard_start, lay.shard_end) if layout == "shard" else (0, n)
    flat = torch.full((n,), float("nan"), device=DEV)
    with_flat = k1(tab, dtype, 0, n, lo, hi, flat=flat, tiles=True)
    without = k1(tab, dtype, 0, n, lo, hi, tiles=True)
    for a, b in zip(with_flat, without):
        np.testing.assert_array_equal(a.view(np.uint8), b.view(np.uint8))
    psum, pflag, tsum, tflag = without
    assert tsum.size == -(-n // _native.SCAN_TILE) and not tflag.any()
    want, _ = _oracle_flat(shapes, grads, 1.0)
    np.testing.assert_array_equal(bits(flat), bits(want))
    owned = want.numpy().copy()
    owned[:lo] = 0.0
    owned[hi:] = 0.0
    T = _native.SCAN_TILE
    for t in range(tsum.size):
        exact = recipe.sumsq_f64(owned[t * T:(t + 1) * T])
        assert abs(tsum[t] - exact) <= 1e-12 * exact, t


def test_k1_owned_range_only_counts_owned_elements():
    shapes = RAGGED
    grads = ragged_grads(shapes, F32, 1e-2, seed=5)
    dg = _device(grads)
    lay, tab = _grad_table(shapes, dg, world=3, rank=1, stage=2)
    n = lay.numel_padded
    lo, hi = lay.shard_start, lay.shard_end
    psum, _ = k1(tab, F32, 0, n, lo, hi)
    flat, _ = _oracle_flat(shapes, grads, 1.0)
    exact = recipe.sumsq_f64(flat.numpy()[lo:hi])
    assert abs(psum.sum() - exact) <= 1e-12 * exact


def test_k2_norm_clip_and_scaler_decisions():
    nb = _native.stats_blocks()
    rng = np.random.default_rng(0)
    psum = rng.random(2 * nb) * 1e-3
    pflag = np.zeros(2 * nb, dtype=np.int32)
    g0 = np.float32(psum[:nb].sum())
    g1 = np.float32(psum[nb:].sum())
    want_sumsq = np.float32(g0 + g1)
    s = k2(psum, pflag, ngroups=2, has_clip=True, max_norm=0.5,
           scaler=(True, 2.0 ** 16, 998, 3, 1000, 1.0, 2.0 ** 24))
    assert abs(int(np.float32(s.sumsq).view(np.int32)) - int(want_sumsq.view(np.int32))) <= 1
    assert np.float32(s.norm) == np.sqrt(np.float32(s.sumsq))
    applied, coef64, coef32 = recipe.clip_coef(s.norm, 0.5)
    assert bool(s.clip_applied) == applied
    assert s.coef64 == coef64 and np.float32(s.coef) == np.float32(coef32)
    assert (s.next_scale, s.next_good_steps, s.next_skipped_steps) == (2.0 ** 16, 999, 3)
    s = k2(psum, pflag, ngroups=2, scaler=(True, 2.0 ** 16, 999, 3, 1000, 1.0, 2.0 ** 24))
    assert (s.next_scale, s.next_good_steps) == (2.0 ** 17, 0)
    assert not s.clip_applied
    s = k2(psum, pflag, ngroups=2, scaler=(True, 2.0 ** 24, 999, 3, 1000, 1.0, 2.0 ** 24))
    assert (s.next_scale, s.next_good_steps) == (2.0 ** 24, 1000)
    pflag[nb + 17] = 1
    s = k2(psum, pflag, ngroups=2, has_clip=True, max_norm=1e-9,
           scaler=(True, 1.0, 5, 3, 1000, 1.0, 2.0 ** 24))
    assert s.overflow and not s.clip_applied
    assert (s.next_scale, s.next_good_steps, s.next_skipped_steps) == (1.0, 0, 4)
    s = k2(psum, pflag, ngroups=1)   # the flag sits in group 1 only
    assert not s.overflow


def _adam_case(shapes, gdtype, seed, scale=1.0, zero_grad_params=()):
    rng = np.random.default_rng(seed)
    lay = layout_for([int(np.prod(s)) for s in shapes])
    n = lay.numel_padded
    p = rng.normal(0, 0.02, n).astype(np.float32)
    m = (rng.normal(0, 1e-3, n)).astype(np.float32)
    v = (rng.random(n) * 1e-6).astype(np.float32)
    grads = ragged_grads(shapes, gdtype, 1e-3, seed=seed + 1, scale=scale)
    for i in zero_grad_params:
        grads[i] = None
    return lay, p, m, v, grads


def _flat_np(lay, grads):
    out = np.zeros(lay.numel_padded, dtype=np.float32)
    for g, off in zip(grads, lay.offsets):
        if g is not None:
            out[off:off + g.numel()] = g.float().reshape(-1).numpy()
    return out


@pytest.mark.parametrize("gdtype", [F16, BF16, F32])
@pytest.mark.parametrize("shapes", [RAGGED, ALIGNED], ids=["ragged", "aligned"])
@pytest.mark.parametrize("variant", ["plain", "unscale_clip_decay", "flat_grad", "late_step"])
def test_k3_matches_kernel_recipe_bitwise(gdtype, shapes, variant):
    scale = 65536.0 if variant == "unscale_clip_decay" and gdtype == F16 else 1.0
    lay, p, m, v, grads = _adam_case(shapes, gdtype, seed=7, scale=scale, zero_grad_params=(1,))
    n = lay.numel_padded
    lr, betas, eps = 1e-3, (0.9, 0.999), 1e-8
    wd = 0.01 if variant in ("unscale_clip_decay", "late_step") else 0.0
    step = 1000 if variant == "late_step" else 3
    clip = 0.37 if variant in ("unscale_clip_decay", "late_step") else None
    dg = _device(grads)
    models = [torch.zeros(s, dtype=gdtype, device=DEV) for s in shapes]
    gst = [store(g, off) for g, off in zip(dg, lay.offsets)]
    mst = [store(t, off) for t, off in zip(models, lay.offsets)]
    flat_grad = None
    unscale = scale != 1.0
    if variant == "flat_grad":
        flat_grad = torch.from_numpy(_flat_np(lay, grads)).to(DEV)
        tab = Table(lay, 0, n, [None] * len(shapes), mst)
    else:
        tab = Table(lay, 0, n, gst, mst)
    dp, dm, dv = (torch.from_numpy(x.copy()).to(DEV) for x in (p, m, v))
    hp = adamw_params(lr, betas, eps, wd, step, grad_scale=scale, unscale=unscale)
    sc = scalars_device(clip_applied=1 if clip else 0, coef=clip or 1.0)
    k3(tab, gdtype, gdtype, 0, n, dp, dm, dv, hp, sc, flat_grad=flat_grad)
    g = _flat_np(lay, grads)
    wp, wm, wv = recipe.adamw_step(p, m, v, g, lr=lr, betas=betas, eps=eps, wd=wd, step=step,
                                   grad_scale=scale, unscale=unscale, clip_coef=clip)
    np.testing.assert_array_equal(dm.cpu().numpy().view(np.int32), wm.view(np.int32))
    np.testing.assert_array_equal(dv.cpu().numpy().view(np.int32), wv.view(np.int32))
    np.testing.assert_array_equal(dp.cpu().numpy().view(np.int32), wp.view(np.int32))
    want_model = torch.from_numpy(wp).to(gdtype)
    got_model = torch.cat([t.reshape(-1).cpu() for t in models])
    np.testing.assert_array_equal(bits(got_model), bits(want_model[:lay.numel]))


@pytest.mark.parametrize("gdtype", [F16, BF16])
def test_k3_against_torch_restatement(gdtype):
    shapes = RAGGED
    lay, p, m, v, grads = _adam_case(shapes, gdtype, seed=9)
    n = lay.numel_padded
    lr, betas, eps, wd, step, coef = 1e-3, (0.9, 0.999), 1e-8, 0.01, 5, 0.41
    dg = _device(grads)
    tab = Table(lay, 0, n, [store(g, off) for g, off in zip(dg, lay.offsets)], [None] * len(shapes))
    dp, dm, dv = (torch.from_numpy(x.copy()).to(DEV) for x in (p, m, v))
    k3(tab, gdtype, gdtype, 0, n, dp, dm, dv, adamw_params(lr, betas, eps, wd, step),
       scalars_device(clip_applied=1, coef=coef))
    tp, tm, tv = (torch.from_numpy(x.copy()) for x in (p, m, v))
    tg = torch.from_numpy(_flat_np(lay, grads))
    tg.mul_(float(np.float32(coef)))
    ob.adam_update(tp, tg, tm, tv, lr, betas, eps, wd, step)
    np.testing.assert_array_equal(dm.cpu().numpy(), tm.numpy())
    np.testing.assert_array_equal(dv.cpu().numpy(), tv.numpy())
    ok, worst, nsq = master_step_within_ulps(p, dp.cpu().numpy(), tp.numpy(), tm.numpy(), tv.numpy(),
                                             lr=lr, betas=betas, eps=eps, wd=wd, step=step)
    assert ok, (worst, nsq)


def test_k3_skips_everything_on_overflow():
    shapes = RAGGED
    lay, p, m, v, grads = _adam_case(shapes, F16, seed=2)
    n = lay.numel_padded
    dg = _device(grads)
    models = [torch.full(s, 7.0, dtype=F16, device=DEV) for s in shapes]
    tab = Table(lay, 0, n, [store(g, off) for g, off in zip(dg, lay.offsets)],
                [store(t, off) for t, off in zip(models, lay.offsets)])
    dp, dm, dv = (torch.from_numpy(x.copy()).to(DEV) for x in (p, m, v))
    k3(tab, F16, F16, 0, n, dp, dm, dv, adamw_params(1e-3, (0.9, 0.999), 1e-8, 0.01, 1),
       scalars_device(overflow=1))
    np.testing.assert_array_equal(dp.cpu().numpy(), p)
    np.testing.assert_array_equal(dm.cpu().numpy(), m)
    np.testing.assert_array_equal(dv.cpu().numpy(), v)
    assert all(bool((t == 7.0).all()) for t in models)


def test_k3_shard_range_with_placeholders():
    """Rank 1 of 3 (ZeRO-3 style): masters/moments hold the owned slice only
    and every model destination is a placeholder of that slice."""
    shapes = RAGGED
    numels = [int(np.prod(s)) for s in shapes]
    lay = layout_for(numels, world_size=3, rank=1, stage=3)
    lo, hi = lay.shard_start, lay.shard_end
    rng = np.random.default_rng(4)
    p = rng.normal(0, 0.02, hi - lo).astype(np.float32)
    m = np.zeros(hi - lo, np.float32)
    v = np.zeros(hi - lo, np.float32)
    grads = ragged_grads(shapes, BF16, 1e-3, seed=8)
    dg = _device(grads)
    holders, mst = [], []
    for off, nn_ in zip(lay.offsets, numels):
        a, b = max(off, lo), min(off + nn_, hi)
        t = torch.zeros(max(0, b - a), dtype=BF16, device=DEV)
        holders.append((a, b, t))
        mst.append((t.data_ptr(), (a, b), 2) if b > a else None)
    tab = Table(lay, lo, hi, [store(g, off) for g, off in zip(dg, lay.offsets)], mst)
    dp, dm, dv = (torch.from_numpy(x.copy()).to(DEV) for x in (p, m, v))
    hp = adamw_params(1e-3, (0.9, 0.999), 1e-8, 0.0, 1)
    k3(tab, BF16, BF16, lo, hi, dp, dm, dv, hp, scalars_device())
    g = _flat_np(lay, grads)[lo:hi]
    wp, _, _ = recipe.adamw_step(p, m, v, g, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, wd=0.0, step=1)
    np.testing.assert_array_equal(dp.cpu().numpy().view(np.int32), wp.view(np.int32))
    want = torch.from_numpy(wp).to(BF16)
    for a, b, t in holders:
        if b > a:
            np.testing.assert_array_equal(bits(t), bits(want[a - lo:b - lo]))


@pytest.mark.parametrize("mdtype", [F16, BF16, F32])
def test_k4_cast_matches_torch_rounding(mdtype):
    rng = np.random.default_rng(1)
    shapes = RAGGED
    lay = layout_for([int(np.prod(s)) for s in shapes])
    n = lay.numel_padded
    flat = (rng.normal(0, 1, n) * np.exp(rng.uniform(-30, 30, n))).astype(np.float32)
    flat[:6] = [65519.0, 65520.0, -1e5, 1e-8, -0.0, 3.0e38]
    flat[6:9] = np.array([1, 0x80001, 0x7F7FFFFF], dtype=np.int32).view(np.float32)
    models = [torch.zeros(s, dtype=mdtype, device=DEV) for s in shapes]
    tab = Table(lay, 0, n, [None] * len(shapes), [store(t, off) for t, off in zip(models, lay.offsets)])
    k4(tab, mdtype, torch.from_numpy(flat).to(DEV), 0, n)
    want = torch.from_numpy(flat[:lay.numel]).to(mdtype)
    got = torch.cat([t.reshape(-1).cpu() for t in models])
    np.testing.assert_array_equal(bits(got), bits(want))


@pytest.mark.parametrize("dtype", [F16, BF16, F32])
@pytest.mark.parametrize("factor", [1e36, -1e36, 3.0, -1.0, -0.5, 0.0])
def test_k1_flags_follow_the_raw_gradients_under_any_factor(dtype, factor):
    """K1 multiplying by a scale_grads factor (MS_SCALE_MULTIPLY): a tile's
    flag is set exactly when one of its raw gradients is inf/nan — also
    where the factor turns finite gradients into inf (|factor| > 1, where
    the kernel tests every word) or an inf into nan (0); with the factor in
    [-1, 1] the flags of the counted elements come from their sums."""
    lib = _native.load()
    tile = _native.SCAN_TILE
    n = 7 * tile + 100
    g = torch.full((n,), 1e3 if dtype == F16 else 1e10, dtype=torch.float32)
    g[::7] *= -1.0
    g[2 * tile + 5] = float("inf")
    g[4 * tile + tile - 1] = float("nan")
    g[6 * tile + 3] = -float("inf")
    dg = g.to(dtype).to(DEV)
    lay = layout_for([n])
    tab = Table(lay, 0, n, [store(dg, 0)], [None])
    nb, nt = _native.stats_blocks(), _native.scan_tiles(n)
    psum = torch.empty(nb, dtype=torch.float64, device=DEV)
    pflag = torch.empty(nb, dtype=torch.int32, device=DEV)
    tsum = torch.empty(nt, dtype=torch.float64, device=DEV)
    tflag = torch.full((nt,), -1, dtype=torch.int32, device=DEV)
    for lo, hi in ((0, n), (tile + 7, 5 * tile)):      # counted everywhere / partly
        _native.check(lib.ms_grad_stats(tab.ptr, tab.nseg, _native.ms_dtype(dtype), 0, n, lo, hi,
                                        _native.SCALE_MULTIPLY, float(np.float32(factor)), None,
                                        tsum.data_ptr(), tflag.data_ptr(), nt, psum.data_ptr(),
                                        pflag.data_ptr(), nb, stream()), "ms_grad_stats")
        torch.cuda.synchronize()
        raw_bad = ~torch.isfinite(dg.float().cpu())
        want = [int(raw_bad[t * tile:(t + 1) * tile].any()) for t in range(nt)]
        assert [int(f != 0) for f in tflag.cpu().tolist()] == want, (lo, hi)


def test_k2_host_copy_equals_device_result_after_an_event():
    """K2's optional host-side output (pinned memory written by the kernel)
    holds the device result, with ``ready`` set, once an event recorded
    after K2 completes."""
    lib = _native.load()
    nb = _native.stats_blocks()
    rng = np.random.default_rng(3)
    ps = torch.from_numpy(rng.random(nb) * 1e-2).to(DEV)
    pf = torch.zeros(nb, dtype=torch.int32, device=DEV)
    out = torch.zeros(_native.SCALARS_BYTES, dtype=torch.uint8, device=DEV)
    host = torch.full((_native.SCALARS_BYTES,), 0xAB, dtype=torch.uint8, pin_memory=True)
    for k, flag in enumerate((0, 1, 0)):
        pf[17] = flag
        ev = torch.cuda.Event()
        rc = lib.ms_norm_clip(ps.data_ptr(), pf.data_ptr(), nb, 1, 1, 0.5, 1, 2.0 ** 16, k, 0, 1000,
                              1.0, 2.0 ** 24, out.data_ptr(), host.data_ptr(), stream())
        _native.check(rc, "ms_norm_clip")
        ev.record()
        ev.synchronize()
        got = _native.StepScalars.from_buffer_copy(host.numpy().tobytes())
        dev = _native.StepScalars.from_buffer_copy(out.cpu().numpy().tobytes())
        assert got.ready == 1 and dev.ready == 0
        dev.ready = 1
        assert bytes(got) == bytes(dev)
        assert got.overflow == flag and got.next_good_steps == (0 if flag else k + 1)


def test_k2_host_result_is_polled_while_later_kernels_run():
    """The engine's read-back: ``ready`` cleared, K2 launched with the
    pinned host output, K3 queued behind it; the host polls ``ready`` and
    then reads the whole struct, equal to the device result, while the
    stream may still be running K3 (HostReadback)."""
    from minispeed_amd.boundary import HostReadback

    lib = _native.load()
    nb = _native.stats_blocks()
    rng = np.random.default_rng(4)
    ps = torch.from_numpy(rng.random(nb) * 1e-2).to(DEV)
    pf = torch.zeros(nb, dtype=torch.int32, device=DEV)
    out = torch.zeros(_native.SCALARS_BYTES, dtype=torch.uint8, device=DEV)
    rb = HostReadback(patience=30.0)
    n = 1 << 24
    lay, p, m, v, grads = _adam_case([(n,)], F16, seed=1)
    tab = Table(lay, 0, n, [store(g, off) for g, off in zip(_device(grads), lay.offsets)], [None])
    dp, dm, dv = (torch.from_numpy(x.copy()).to(DEV) for x in (p, m, v))
    lib_k3 = lib.ms_fused_adamw
    for k, flag in enumerate((0, 1, 0, 0)):
        pf[123] = flag
        torch.cuda.synchronize()
        rb.arm()
        assert rb.host.numpy()[_native.StepScalars.ready.offset] == 0
        rc = lib.ms_norm_clip(ps.data_ptr(), pf.data_ptr(), nb, 1, 1, 0.5, 1, 2.0 ** 16, k, 0, 1000,
                              1.0, 2.0 ** 24, out.data_ptr(), rb.ptr, stream())
        _native.check(rc, "ms_norm_clip")
        hp = adamw_params(1e-3, (0.9, 0.999), 1e-8, 0.01, k + 1)
        _native.check(lib_k3(dp.data_ptr(), dm.data_ptr(), dv.data_ptr(), None, tab.ptr, tab.nseg,
                             _native.ms_dtype(F16), _native.ms_dtype(F16), 0, n, ctypes.byref(hp),
                             out.data_ptr(), stream()), "ms_fused_adamw")
        got = rb.wait(stream())
        torch.cuda.synchronize()
        dev = _native.StepScalars.from_buffer_copy(out.cpu().numpy().tobytes())
        assert got.ready == 1
        dev.ready = 1
        assert bytes(got) == bytes(dev), k
        assert got.overflow == flag


def test_boundary_kernels_replay_in_a_hip_graph():
    """K1 -> K2 -> K3 captured once in a graph and replayed from the same
    starting state several times, with eager work and synchronisations in
    between, gives the eager result every time (no memset nodes, no host
    sync inside; K1 zero-fills its partial slots itself)."""
    lib = _native.load()
    shapes = RAGGED
    grads = _device(ragged_grads(shapes, F16, 1e-2, seed=77, scale=1024.0))
    lay = layout_for([int(np.prod(s)) for s in shapes])
    n = lay.numel_padded
    models = [torch.empty(int(np.prod(s)), dtype=F16, device=DEV) for s in shapes]
    table = Table(lay, 0, n, [store(g, off) for g, off in zip(grads, lay.offsets)],
                  [store(m, off) for m, off in zip(models, lay.offsets)])
    nb = _native.stats_blocks()
    psum = torch.empty(nb, dtype=torch.float64, device=DEV)
    pflag = torch.empty(nb, dtype=torch.int32, device=DEV)
    nt = _native.scan_tiles(n)
    tsum = torch.empty(nt, dtype=torch.float64, device=DEV)
    tflag = torch.empty(nt, dtype=torch.int32, device=DEV)
    scal = torch.empty(_native.SCALARS_BYTES, dtype=torch.uint8, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(3)
    p0 = torch.randn(n, generator=gen, device=DEV) * 0.02
    m0 = torch.randn(n, generator=gen, device=DEV) * 1e-3
    v0 = torch.rand(n, generator=gen, device=DEV) * 1e-6
    p, m, v = p0.clone(), m0.clone(), v0.clone()
    hp = adamw_params(1e-3, (0.9, 0.999), 1e-8, 0.01, 7, grad_scale=1024.0, unscale=True)

    def boundary(st):
        _native.check(lib.ms_grad_stats(table.ptr, table.nseg, _native.DTYPE_F16, 0, n, 0, n, 1,
                                        1024.0, None, tsum.data_ptr(), tflag.data_ptr(), nt,
                                        psum.data_ptr(), pflag.data_ptr(), nb, st), "k1")
        _native.check(lib.ms_norm_clip(psum.data_ptr(), pflag.data_ptr(), nb, 1, 1, 0.5, 1, 1024.0,
                                       3, 0, 1000, 1.0, 2.0 ** 24, scal.data_ptr(), None, st), "k2")
        _native.check(lib.ms_fused_adamw(p.data_ptr(), m.data_ptr(), v.data_ptr(), None, table.ptr,
                                         table.nseg, _native.DTYPE_F16, _native.DTYPE_F16, 0, n,
                                         ctypes.byref(hp), scal.data_ptr(), st), "k3")

    boundary(stream())
    torch.cuda.synchronize()
    want = [t.clone() for t in (p, m, v, scal)] + [torch.cat(models).clone()]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        for t, t0 in ((p, p0), (m, m0), (v, v0)):
            t.copy_(t0)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            boundary(side.cuda_stream)
    torch.cuda.synchronize()
    for rep in range(4):
        for t, t0 in ((p, p0), (m, m0), (v, v0)):
            t.copy_(t0)
        psum.fill_(float("nan"))          # eager work between replays
        scal.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [p, m, v, scal, torch.cat(models)]
        for a, b in zip(got, want):
            assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), rep


@pytest.mark.parametrize("seed", range(6))
def test_random_layouts_with_misaligned_views_and_empty_params(seed):
    """Random ragged lists (some zero-size), every gradient and model copy a
    view at a random element offset of one pool (so most addresses are not
    16-byte aligned), a random owned range: K1's flags / sum of squares /
    flat gradient, K3 against the recipe bit for bit (elements outside the
    range untouched) and K4's casts against torch."""
    rng = np.random.default_rng(100 + seed)
    gdtype = [F16, BF16, F32][seed % 3]
    sizes = [int(x) for x in rng.integers(0, 3000, size=14)]
    sizes[int(rng.integers(0, 14))] = 0
    sizes[0] = max(sizes[0], 1)
    lay = layout_for(sizes)
    n = lay.numel_padded
    lo = int(rng.integers(0, n // 3))
    hi = int(rng.integers(2 * n // 3, n + 1))
    gen = torch.Generator().manual_seed(seed)

    def pool_views(dtype, fill):
        pool = torch.full((sum(sizes) + 8 * len(sizes) + 8,), fill, dtype=dtype, device=DEV)
        views, pos = [], int(rng.integers(0, 8))
        for k in sizes:
            views.append(pool[pos:pos + k])
            pos += k + int(rng.integers(0, 8))
        return pool, views

    gpool, gviews = pool_views(gdtype, 0.0)
    grads_cpu = []
    for view, k in zip(gviews, sizes):
        gcpu = (torch.randn(k, generator=gen) * 1e-2).to(gdtype)
        view.copy_(gcpu.to(DEV))
        grads_cpu.append(gcpu)
    if seed == 4 and sizes[3] > 0:
        gviews[3][0] = float("nan")
        grads_cpu[3][0] = float("nan")
    gst = [(v.data_ptr(), (off, off + k), v.element_size()) if k else None
           for v, off, k in zip(gviews, lay.offsets, sizes)]
    flat_want = np.zeros(n, np.float32)
    for gcpu, off, k in zip(grads_cpu, lay.offsets, sizes):
        flat_want[off:off + k] = gcpu.float().numpy()

    # K1: flat gradient, flags, owned-range sum of squares
    tab1 = Table(lay, 0, n, gst, [None] * len(sizes))
    flat = torch.full((n,), 7.0, device=DEV)
    psum, pflag = k1(tab1, gdtype, 0, n, lo, hi, flat=flat)
    np.testing.assert_array_equal(flat.cpu().numpy().view(np.int32), flat_want.view(np.int32))
    assert bool(pflag.any()) == (seed == 4 and sizes[3] > 0)
    if seed != 4:
        exact = recipe.sumsq_f64(flat_want[lo:hi])
        assert abs(psum.sum() - exact) <= 1e-12 * max(exact, 1e-300)
        # K3 over [lo, hi) with misaligned model copies
        mpool, mviews = pool_views(gdtype, 3.0)
        mst = [(v.data_ptr(), (off, off + k), v.element_size()) if k else None
               for v, off, k in zip(mviews, lay.offsets, sizes)]
        tab3 = Table(lay, lo, hi, gst, mst)
        p = rng.normal(0, 0.02, hi - lo).astype(np.float32)
        m = rng.normal(0, 1e-3, hi - lo).astype(np.float32)
        v = np.abs(rng.normal(0, 1e-6, hi - lo)).astype(np.float32)
        dp, dm, dv = (torch.from_numpy(x.copy()).to(DEV) for x in (p, m, v))
        hp = adamw_params(1e-3, (0.9, 0.999), 1e-8, 0.01, 4)
        k3(tab3, gdtype, gdtype, lo, hi, dp, dm, dv, hp, scalars_device(clip_applied=1, coef=0.7))
        wp, wm, wv = recipe.adamw_step(p, m, v, flat_want[lo:hi], lr=1e-3, betas=(0.9, 0.999),
                                       eps=1e-8, wd=0.01, step=4, clip_coef=0.7)
        np.testing.assert_array_equal(dp.cpu().numpy().view(np.int32), wp.view(np.int32))
        np.testing.assert_array_equal(dm.cpu().numpy().view(np.int32), wm.view(np.int32))
        np.testing.assert_array_equal(dv.cpu().numpy().view(np.int32), wv.view(np.int32))
        cast = torch.from_numpy(wp).to(gdtype)
        for view, off, k in zip(mviews, lay.offsets, sizes):
            got = view.cpu()
            a, b = max(off, lo), min(off + k, hi)
            for i0, i1 in ((off, a), (b, off + k)):           # outside the range: untouched
                if i1 > i0:
                    assert bool((got[i0 - off:i1 - off] == 3.0).all())
            if b > a:
                np.testing.assert_array_equal(bits(got[a - off:b - off]), bits(cast[a - lo:b - lo]))
        # K4 over the same range into the same views
        src = rng.normal(0, 1, hi - lo).astype(np.float32)
        k4(Table(lay, lo, hi, [None] * len(sizes), mst), gdtype, torch.from_numpy(src).to(DEV), lo, hi)
        want4 = torch.from_numpy(src).to(gdtype)
        for view, off, k in zip(mviews, lay.offsets, sizes):
            a, b = max(off, lo), min(off + k, hi)
            if b > a:
                np.testing.assert_array_equal(bits(view.cpu()[a - off:b - off]),
                                              bits(want4[a - lo:b - lo]))


# The reading K1 takes the runs holding the last 224 MiB of gradient with
# ordinary loads (K3 then finds those lines in the Infinity Cache) and the
# other runs with non-temporal loads; the writing K1 never keeps anything.
KEEP_BYTES = 224 << 20


@pytest.mark.parametrize("dtype", [F16, BF16, F32])
def test_k1_cache_keeping_runs_match_the_writing_scan(dtype):
    """A layout past the keeping threshold, so that both kinds of run are
    scanned: the reading and the writing K1 give the same tile sums and
    flags bit for bit, the sums match exact fp64 sums of squares of the
    unscaled values K1 wrote, and an inf / nan planted in a non-temporal run
    and in a kept run flags exactly its tile."""
    esize = torch.empty(0, dtype=dtype).element_size()
    keep_tiles = KEEP_BYTES // (_native.SCAN_TILE * esize)
    n_want = (keep_tiles + 3000) * _native.SCAN_TILE
    shapes = [(n_want // 3 - 5,), (n_want // 3 + 11,), (n_want - 2 * (n_want // 3) + 7,)]
    gen = torch.Generator(device=DEV).manual_seed(11)
    grads = [(torch.randn(*s, generator=gen, device=DEV) * 1e-2).to(dtype) for s in shapes]
    lay, tab = _grad_table(shapes, grads)
    n = lay.numel_padded
    scale = 65536.0 if dtype == F16 else 1.0
    if scale != 1.0:
        for g in grads:
            g.mul_(scale)
    _, _, ts_read, tf_read = k1(tab, dtype, 0, n, 0, n, scale=scale, tiles=True)
    flat = torch.full((n,), float("nan"), dtype=torch.float32, device=DEV)
    _, _, ts_write, tf_write = k1(tab, dtype, 0, n, 0, n, scale=scale, flat=flat, tiles=True)
    nt = ts_read.size
    assert nt > keep_tiles + 1000
    np.testing.assert_array_equal(ts_read.view(np.int64), ts_write.view(np.int64))
    np.testing.assert_array_equal(tf_read, tf_write)
    assert not tf_read.any()
    want = torch.cat([g.float().reshape(-1) for g in grads]).div_(scale)
    got = flat[:want.numel()]
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))
    x = flat.cpu().numpy().astype(np.float64)
    x[want.numel():] = 0.0
    pad = nt * _native.SCAN_TILE - n
    exact = np.pad(x * x, (0, pad)).reshape(nt, _native.SCAN_TILE).sum(axis=1)
    np.testing.assert_allclose(ts_read, exact, rtol=1e-12, atol=0)
    # one special value in a non-temporal run (first third) and one in a kept run (the end)
    special = {torch.float16: (0x7C00, 0x7E00), torch.bfloat16: (0x7F80, 0x7FC0),
               torch.float32: (0x7F800000, 0x7FC00000)}[dtype]
    i0, i1 = 12_345, n_want - 17
    lo_tile, hi_tile = (lay.offsets[0] + i0) // _native.SCAN_TILE, None
    set_bits(grads[0], i0, special[0])
    last = grads[2]
    set_bits(last, last.numel() - 17, special[1])
    hi_tile = (lay.offsets[2] + last.numel() - 17) // _native.SCAN_TILE
    assert lo_tile < nt - keep_tiles - 4 and hi_tile >= nt - keep_tiles
    _, _, _, tf = k1(tab, dtype, 0, n, 0, n, scale=scale, tiles=True)
    assert set(np.flatnonzero(tf)) == {lo_tile, hi_tile}
