"""Opt-in contiguous gradients on the GPU.

* K5 (``ms_accumulate_grad``, and batched, ``ms_accumulate_grads``: 150
  rows, three launches) against the fp32 sum of widened gradients, bit for
  bit, for every dtype, aligned and misaligned slices, ragged sizes,
  inf/nan; the elements between the slices stay untouched;
* the engine in this mode against the oracle's boundary given the fp32 sums
  (bit-exact flags, scale and Adam moments when the clip coefficients agree;
  masters within 2 fp32 ulp per step; norm within 1e-5), through real
  backward passes with gradient accumulation;
* where half-precision accumulation is exact the mode equals the default
  mode bit for bit; parameters without a gradient in a window count as
  zeros; an overflow skips the step and the next window starts clean;
  ZeRO-3 equals ZeRO-0; flushing the queued gradients inside backward (a
  bucket of one element) equals one flush at the end of backward;
* the boundary from K5's tile statistics (``ms_reduce_tile_stats``, checked
  on its own against in-order fp64 sums) against the boundary that scans
  the sums again, and the fall-back to that scan when the loss scale
  changed inside a window.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch
from torch import nn

import minispeed_amd as ms
from minispeed_amd import _native
from oracle import boundary as ob
from tests.helpers import clip_override, master_step_within_ulps, step_hyper

pytestmark = pytest.mark.gpu
DEV = "cuda"
SHAPES = [(7, 5), (3,), (16, 33), (1,), (129,), (64, 8)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n,off", [(1, 0), (7, 3), (8, 4), (2049, 1), (100003, 8), (65536, 0)])
def test_accumulate_kernel_is_the_fp32_sum(dtype, n, off):
    lib = _native.load()
    g = torch.Generator(device=DEV).manual_seed(n + off)
    parts = [torch.randn(n, generator=g, device=DEV).to(dtype) for _ in range(3)]
    if n > 10:
        parts[1][5] = float("inf")
        parts[2][9] = float("nan")
    buf = torch.full((n + off + 8,), -3.0, device=DEV)
    dst = buf.data_ptr() + off * 4
    stream = _native.stream_handle(torch.device(DEV))
    want = None
    for k, x in enumerate(parts):
        _native.check(lib.ms_accumulate_grad(dst, x.data_ptr(), _native.ms_dtype(dtype), n,
                                             1 if k == 0 else 0, stream), "ms_accumulate_grad")
        want = ob.accumulate_fp32(want, x.cpu())
        got = buf[off:off + n].cpu()
        assert torch.equal(got.view(torch.int32)[~torch.isnan(want)],
                           want.view(torch.int32)[~torch.isnan(want)]), k
        assert torch.equal(torch.isnan(got), torch.isnan(want))
    # the guard elements around the slice are untouched
    assert torch.all(buf[:off].cpu() == -3.0) and torch.all(buf[off + n:].cpu() == -3.0)


@pytest.mark.parametrize("dtype,scale_value", [(torch.float16, 1024.0), (torch.bfloat16, 1000.0),
                                               (torch.float32, 3.0)])
def test_batched_accumulation_is_the_fp32_sum_of_every_row(dtype, scale_value):
    """150 rows (three launches of 64 / 64 / 22) of ragged sizes, dst slices
    at every alignment with 3 guard elements between them, some sources one
    element off their alignment, first / add mixed within a launch; the
    tile statistics of the new sums against fp64 on the CPU (power-of-two
    and IEEE-division unscaling), rows without slots leave them alone."""
    from minispeed_amd.contiguous import ACCUM_ROW, accumulate_rows
    rng = np.random.default_rng(7)
    sizes = rng.choice([0, 1, 3, 4, 2047, 2048, 2049, 4101, 10000], size=150)
    shifts = rng.integers(0, 4, size=150)          # dst start mod 4
    pos, p = [], 8
    for n, sh in zip(sizes, shifts):
        p += (-p + sh) % 4
        pos.append(p)
        p += int(n) + 3
    buf = torch.full((p + 8,), -3.0, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(11)
    want = [None] * len(sizes)
    tiles = [(int(n) + 2047) // 2048 for n in sizes]
    t0 = np.concatenate([[0], np.cumsum(tiles)[:-1]]).astype(np.int64)
    ts = torch.empty(max(1, sum(tiles)), dtype=torch.float64, device=DEV)
    tf = torch.empty(max(1, sum(tiles)), dtype=torch.int32, device=DEV)
    unscale, scale = _native.SCALE_DIVIDE, scale_value
    for rnd in range(3):
        srcs, rows = [], np.zeros(len(sizes), dtype=ACCUM_ROW)
        for r, n in enumerate(sizes):
            off = int(rng.integers(0, 2)) if rnd else 0
            x = torch.randn(int(n) + off, generator=gen, device=DEV).to(dtype)[off:]
            if n > 100 and rnd == 1 and r % 7 == 0:
                x[17] = float("inf")
                x[40] = float("nan")
            srcs.append(x)
            first = rnd == 0 or (rnd == 2 and r % 5 == 0)
            stats = r % 3 != 2                      # some rows without statistics slots
            rows[r] = (buf.data_ptr() + 4 * pos[r], x.data_ptr(), int(n), 1 if first else 0, 0,
                       ts.data_ptr() + 8 * t0[r] if stats else 0,
                       tf.data_ptr() + 4 * t0[r] if stats else 0)
            want[r] = ob.accumulate_fp32(None if first else want[r], x.cpu())
        ts.fill_(-1.0)
        tf.fill_(-1)
        accumulate_rows(rows, _native.ms_dtype(dtype), torch.device(DEV), unscale, scale)
        host, hts, htf = buf.cpu(), ts.cpu().numpy(), tf.cpu().numpy()
        for r, n in enumerate(sizes):
            got, w = host[pos[r]:pos[r] + int(n)], want[r]
            ok = ~torch.isnan(w)
            assert torch.equal(got.view(torch.int32)[ok], w.view(torch.int32)[ok]), (rnd, r)
            assert torch.equal(torch.isnan(got), torch.isnan(w)), (rnd, r)
            # per 2048-element tile: fp64 sum of squares of the unscaled new
            # sums (the boundary scan's unscale) and the inf/nan flag
            for k in range(tiles[r]):
                seg = w[k * 2048:(k + 1) * 2048]
                slot = t0[r] + k
                if r % 3 == 2:
                    assert hts[slot] == -1.0 and htf[slot] == -1, (rnd, r, k)   # untouched
                    continue
                bad = not bool(torch.isfinite(seg).all())
                assert (htf[slot] != 0) == bad, (rnd, r, k)
                if not bad:
                    u = (seg / np.float32(scale)) if unscale else seg
                    ref = float(np.sum(u.double().numpy() ** 2))
                    assert abs(hts[slot] - ref) <= 1e-12 * ref, (rnd, r, k, hts[slot], ref)
        touched = torch.zeros(len(host), dtype=torch.bool)
        for r, n in enumerate(sizes):
            touched[pos[r]:pos[r] + int(n)] = True
        assert torch.all(host[~touched] == -3.0), rnd


def _wave_fold(x: np.ndarray) -> float:
    """The fold's order for one slot: lane l adds x[l], x[l + 64], ... in
    order, then the xor tree (off 32, 16, ..., 1) adds the lanes."""
    lanes = np.array([np.cumsum(x[lane::64])[-1] if len(x) > lane else 0.0 for lane in range(64)])
    off = 32
    while off:
        lanes = lanes + lanes[np.arange(64) ^ off]
        off //= 2
    return float(lanes[0])


def test_folding_tile_statistics_sums_fixed_ranges_in_order():
    """ms_reduce_tile_stats: slot j is the fixed-order fp64 sum of tiles
    [j*T/nb, (j+1)*T/nb) and the OR of their flags, every slot written."""
    lib = _native.load()
    nb = _native.stats_blocks()
    stream = _native.stream_handle(torch.device(DEV))
    rng = np.random.default_rng(5)
    for ntiles in (0, 1, 7, nb - 3, nb, 100_003, 3 * nb + 70 * 64 + 5, 130 * nb):
        ts_h = rng.standard_normal(ntiles) ** 2 * 10.0 ** rng.integers(-8, 8, ntiles)
        tf_h = (rng.random(ntiles) < 0.001).astype(np.int32)
        ts = torch.from_numpy(ts_h).to(DEV)
        tf = torch.from_numpy(tf_h).to(DEV)
        bs = torch.full((nb,), -1.0, dtype=torch.float64, device=DEV)
        bf = torch.full((nb,), 7, dtype=torch.int32, device=DEV)
        _native.check(lib.ms_reduce_tile_stats(ts.data_ptr() if ntiles else None,
                                               tf.data_ptr() if ntiles else None, ntiles,
                                               bs.data_ptr(), bf.data_ptr(), nb, stream),
                      "ms_reduce_tile_stats")
        got_s, got_f = bs.cpu().numpy(), bf.cpu().numpy()
        for j in range(nb):
            lo, hi = j * ntiles // nb, (j + 1) * ntiles // nb
            want = _wave_fold(ts_h[lo:hi])
            assert got_s[j] == want, (ntiles, j)
            assert got_f[j] == (1 if tf_h[lo:hi].any() else 0), (ntiles, j)


def test_accumulate_kernel_rejects_bad_arguments():
    lib = _native.load()
    x = torch.zeros(4, device=DEV)
    assert lib.ms_accumulate_grad(None, x.data_ptr(), 0, 4, 1, None) == -1
    assert lib.ms_accumulate_grad(x.data_ptr(), x.data_ptr(), 7, 4, 1, None) == -1
    assert lib.ms_accumulate_grad(x.data_ptr(), x.data_ptr(), 0, -1, 1, None) == -1
    assert lib.ms_accumulate_grad(x.data_ptr(), x.data_ptr(), 0, 0, 1, None) == 0


class Linear(nn.Module):
    """loss = sum_k sum(p_k * c_k): d loss / d p_k = c_k exactly."""

    def __init__(self, dtype):
        super().__init__()
        g = torch.Generator().manual_seed(3)
        self.ps = nn.ParameterList(nn.Parameter((torch.randn(*s, generator=g) * 0.05).to(dtype))
                                   for s in SHAPES)

    def forward(self, cs, skip=()):
        return sum((p.float() * c).sum() for k, (p, c) in enumerate(zip(self.ps, cs))
                   if k not in skip)


def _cfg(dtype, stage=0, contiguous=True, gas=2):
    cfg = {"train_micro_batch_size_per_gpu": 1, "gradient_accumulation_steps": gas,
           "gradient_clipping": 1.0, "dtype": dtype,
           "optimizer": {"type": "AdamW", "params": {"lr": 1e-2, "weight_decay": 0.01}},
           "zero_optimization": {"stage": stage},
           "hip_boundary": {"contiguous_gradients": contiguous}}
    if dtype == "fp16":
        cfg["fp16"] = {"enabled": True, "loss_scale": 0, "initial_scale_power": 8,
                       "loss_scale_window": 1000}
    return cfg


def _coeffs(seed, dyadic):
    g = torch.Generator().manual_seed(seed)
    out = []
    for s in SHAPES:
        c = torch.randn(*s, generator=g)
        if dyadic:
            c = torch.round(c * 16) / 16          # few significant bits: exact in half
        out.append(c.to(DEV))
    return out


def _run(dtype, stage, contiguous, windows, dyadic, skip_at=None, inf_at=None, gas=2, bucket=None):
    torch.manual_seed(0)
    model = Linear({"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[dtype]).to(DEV)
    engine = ms.initialize(model=model, model_parameters=list(model.parameters()),
                           config=_cfg(dtype, stage, contiguous, gas))
    if bucket is not None:
        engine.contiguous.bucket_elements = bucket
    applied = []
    for w in range(windows):
        for m in range(gas):
            skip = (2,) if skip_at == w else ()
            cs = _coeffs(100 * w + m, dyadic)
            if inf_at == (w, m):
                cs[0].view(-1)[0] = float("inf")   # the first parameter's gradient gets an inf
            loss = engine(cs, skip)
            engine.backward(loss)
            if contiguous:
                assert all(p.grad is None for p in model.parameters())
            applied.append(engine.step())
    return engine, model, applied


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
def test_equals_default_mode_where_half_accumulation_is_exact(dtype):
    a, ma, ra = _run(dtype, 0, False, 4, dyadic=True)
    b, mb, rb = _run(dtype, 0, True, 4, dyadic=True)
    assert ra == rb
    assert a.grad_norm == b.grad_norm and a.get_loss_scale() == b.get_loss_scale()
    assert torch.equal(a.flat_groups[0].data, b.flat_groups[0].data)
    assert torch.equal(a.optimizer.state[0]["exp_avg_sq"], b.optimizer.state[0]["exp_avg_sq"])


def test_missing_gradients_count_as_zero_and_do_not_leak_from_earlier_windows():
    a, _, _ = _run("bf16", 0, False, 3, dyadic=True, skip_at=1)
    b, _, _ = _run("bf16", 0, True, 3, dyadic=True, skip_at=1)
    assert torch.equal(a.flat_groups[0].data, b.flat_groups[0].data)
    assert a.grad_norm == b.grad_norm


def test_overflow_skips_and_the_next_window_starts_clean():
    a, _, ra = _run("fp16", 0, False, 3, dyadic=True, inf_at=(1, 1))
    b, _, rb = _run("fp16", 0, True, 3, dyadic=True, inf_at=(1, 1))
    assert ra == rb and rb.count(True) == 2 and b.skipped_steps == 1
    assert a.get_loss_scale() == b.get_loss_scale() == 2.0 ** 7
    assert torch.equal(a.flat_groups[0].data, b.flat_groups[0].data)


def test_flushes_inside_backward_equal_one_flush_at_its_end():
    a, _, ra = _run("bf16", 0, True, 3, dyadic=False, gas=3)
    b, _, rb = _run("bf16", 0, True, 3, dyadic=False, gas=3, bucket=1)
    assert ra == rb
    assert a.grad_norm == b.grad_norm
    assert torch.equal(a.flat_groups[0].data, b.flat_groups[0].data)
    assert torch.equal(a.optimizer.state[0]["exp_avg_sq"], b.optimizer.state[0]["exp_avg_sq"])


def _engine(dtype, gas, bucket=None):
    torch.manual_seed(0)
    model = Linear({"fp16": torch.float16, "bf16": torch.bfloat16}[dtype]).to(DEV)
    engine = ms.initialize(model=model, model_parameters=list(model.parameters()),
                           config=_cfg(dtype, 0, True, gas))
    if bucket is not None:
        engine.contiguous.bucket_elements = bucket
    return engine, model


def _windows(engine, gas, windows, start=0, dyadic=False):
    applied = []
    for w in range(start, start + windows):
        for m in range(gas):
            engine.backward(engine(_coeffs(100 * w + m, dyadic)))
            applied.append(engine.step())
    return applied


@pytest.mark.parametrize("dtype,bucket", [("fp16", None), ("bf16", None), ("fp16", 1)])
def test_tile_statistics_give_the_boundary_of_a_scan_of_the_sums(dtype, bucket):
    """The boundary from K5's tile statistics (folded, no second read of
    the sums) against the boundary that scans the sums with K1: same
    decisions and scale, the same fp32 norm (fp64 partial sums in two
    partitions), the same masters and moments."""
    a, _ = _engine(dtype, 3, bucket)
    b, _ = _engine(dtype, 3, bucket)
    b.contiguous.use_tile_stats = False
    used = []
    orig = a.contiguous.tile_stats

    def spy(gi, scale):
        r = orig(gi, scale)
        used.append(r is not None)
        return r
    a.contiguous.tile_stats = spy
    for w in range(4):
        ra, rb = _windows(a, 3, 1, start=w), _windows(b, 3, 1, start=w)
        assert ra == rb
        assert a.get_loss_scale() == b.get_loss_scale()
        assert abs(a.grad_norm - b.grad_norm) <= 1.2e-7 * b.grad_norm, (w, a.grad_norm, b.grad_norm)
        if a.grad_norm == b.grad_norm:
            assert torch.equal(a.flat_groups[0].data, b.flat_groups[0].data)
            assert torch.equal(a.optimizer.state[0]["exp_avg_sq"], b.optimizer.state[0]["exp_avg_sq"])
    assert used and all(used)


def test_a_loss_scale_change_inside_a_window_falls_back_to_scanning_the_sums():
    a, _ = _engine("fp16", 2)
    b, _ = _engine("fp16", 2)
    b.contiguous.use_tile_stats = False
    scales = iter([a.loss_scaler.loss_scale_factor, 2 * a.loss_scaler.loss_scale_factor])
    a.contiguous.scale_fn = lambda: next(scales)     # the two flushes unscale differently
    for m in range(2):
        a.backward(a(_coeffs(m, False)))
        b.backward(b(_coeffs(m, False)))
    assert a.contiguous.tile_stats(0, a.loss_scaler.loss_scale_factor) is None
    assert a.step() is True and b.step() is True
    assert a.grad_norm == b.grad_norm
    assert torch.equal(a.flat_groups[0].data, b.flat_groups[0].data)


def test_stage3_equals_stage0():
    a, _, _ = _run("fp16", 0, True, 3, dyadic=False)
    b, _, _ = _run("fp16", 3, True, 3, dyadic=False)
    assert torch.equal(a.flat_groups[0].data, b.flat_groups[0].data)
    assert a.grad_norm == b.grad_norm


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_matches_the_oracle_given_the_fp32_sums(dtype):
    """Non-dyadic gradients: fp32 sums differ from half sums; each boundary
    is checked against the oracle started from the GPU's state."""
    tdt = {"fp16": torch.float16, "bf16": torch.bfloat16}[dtype]
    torch.manual_seed(0)
    model = Linear(tdt).to(DEV)
    engine = ms.initialize(model=model, model_parameters=list(model.parameters()),
                           config=_cfg(dtype, 0, True, gas=3))
    ref_params = [nn.Parameter(p.detach().cpu().clone()) for p in model.parameters()]
    ref = ob.Engine([ref_params], [{"lr": 1e-2, "betas": (0.9, 0.999), "eps": 1e-8,
                                    "weight_decay": 0.01}], dtype=dtype, zero_stage=0, clip=1.0,
                    initial_scale_power=8, loss_scale_window=1000)
    g = engine.flat_groups[0]
    differs = False
    for w in range(4):
        sums = [None] * len(SHAPES)
        for m in range(3):
            cs = _coeffs(10 * w + m, dyadic=False)
            loss = engine(cs)
            engine.backward(loss)
            factor = engine.loss_scaler.loss_scale_factor / 3
            # the gradient autograd hands the hook: the engine casts the
            # floating inputs to the parameter dtype, the product rounds in
            # fp32, and the backward of p.float() rounds to the parameter dtype
            for k, c in enumerate(cs):
                c_in = c.cpu().to(tdt).float()
                sums[k] = ob.accumulate_fp32(sums[k], (c_in * np.float32(factor)).to(tdt))
        flat = torch.zeros(g.numel_padded)
        for off, s in zip(g.layout.offsets, sums):
            flat[off:off + s.numel()] = s
        before = g.data.detach().cpu()
        st = engine.optimizer.state[0]
        ref.load_state([before], [st["exp_avg"].cpu()], [st["exp_avg_sq"].cpu()], [st["step"]],
                       (engine.loss_scaler.scale, engine.loss_scaler.good_steps,
                        engine.loss_scaler.skipped_steps),
                       engine.lr_scheduler.last_epoch,
                       [pg["lr"] for pg in engine.optimizer.param_groups])
        ref.micro_steps += 3
        hp = step_hyper(engine)
        assert engine.step() is True
        assert ref.step(flat_grads=[flat], clip_override=clip_override(engine)) is True
        assert abs(engine.grad_norm - ref.grad_norm) <= 1e-5 * ref.grad_norm
        ok, worst, nsq = master_step_within_ulps(before.numpy(), g.data.cpu().numpy(),
                                                 ref.groups[0].data.numpy(), st["exp_avg"].cpu().numpy(),
                                                 st["exp_avg_sq"].cpu().numpy(), **hp)
        assert ok, (w, worst, nsq)
        assert torch.equal(st["exp_avg"].cpu(), ref.state[0]["exp_avg"])
        assert torch.equal(st["exp_avg_sq"].cpu(), ref.state[0]["exp_avg_sq"])
        # the fp32 sums are not half values: half accumulation would differ
        differs = differs or not torch.equal(sums[2].to(tdt).float(), sums[2])
    assert differs
