"""K1 over seeded random ragged layouts, through the C ABI.

Each case draws a ragged list of gradients (odd sizes, exact multiples of
the tile, single elements), drops some gradients (NULL rows), stores some
2-byte / 4-byte aligned only (the per-element path), scans a range
[begin, end) that may start and end inside parameters (K1's tiles are
relative to begin), counts an owned sub-range, scales by one of the four
rules (none; / a power of two, done as a multiply by its reciprocal; / any
other scale, IEEE division; * a factor, scale_grads' rule), and sometimes
plants inf / nan.  Against torch on the CPU (flatten_grads, flat.py:196-213;
unscale_grads, flat.py:243-247; scale_grads, flat.py:249-257; isfinite,
precision.py:79-87):

* the flat gradient over [begin, end) bit for bit (NaNs as NaNs);
* tile t's flag exactly (an inf/nan among its stored, pre-scaling values),
  and its fp64 sum within 1e-12 of the exact sum of squares of its owned,
  scaled elements;
* the partial slots exactly the fold of the tiles (slot j: tiles
  [j*T/nblk, (j+1)*T/nblk)), sums within 1e-12;
* the statistics bit for bit the same without the flat output.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from minispeed_amd import _native
from oracle import recipe
from tests.helpers import DEV, Table, bits, layout_for, store, stream

pytestmark = pytest.mark.gpu

TILE = _native.SCAN_TILE
DTYPES = [torch.float16, torch.bfloat16, torch.float32]
NONFINITE = {torch.float16: [0x7C00, 0xFC00, 0x7E01], torch.bfloat16: [0x7F80, 0xFF80, 0x7FC1],
             torch.float32: [0x7F800000, 0xFF800000, 0x7FC00001]}


def _case(seed):
    rng = np.random.default_rng(seed)
    dtype = DTYPES[seed % 3]
    kinds = rng.integers(0, 4, size=int(rng.integers(1, 24)))
    numels = [int(rng.integers(1, 40)) if k == 0 else
              int(rng.integers(1, 5)) * TILE if k == 1 else
              int(rng.integers(40, 9000)) if k == 2 else
              int(rng.integers(9000, 30000)) for k in kinds]
    host = []
    for n in numels:
        x = torch.from_numpy(rng.standard_normal(n).astype(np.float32) * 1e-3)
        host.append(x.to(dtype))
    if seed % 4 == 3:                                  # plant inf / nan
        for _ in range(int(rng.integers(1, 4))):
            k = int(rng.integers(0, len(host)))
            i = int(rng.integers(0, numels[k]))
            pat = NONFINITE[dtype][int(rng.integers(0, 3))]
            v = host[k].view(torch.int16 if dtype != torch.float32 else torch.int32)
            v[i] = int(np.array(pat, dtype=np.uint32).astype(
                np.int16 if dtype != torch.float32 else np.int32))
    missing = rng.random(len(host)) < 0.15
    misaligned = rng.random(len(host)) < 0.25
    return rng, dtype, numels, host, missing, misaligned


def _device(host, missing, misaligned, dtype):
    out = []
    for x, miss, mis in zip(host, missing, misaligned):
        if miss:
            out.append(None)
        elif mis:
            base = torch.zeros(x.numel() + 1, dtype=dtype, device=DEV)
            base[1:].copy_(x.to(DEV))
            out.append(base[1:])
        else:
            out.append(x.to(DEV))
    return out


def _scaling(rng):
    """(MS_SCALE_* mode, fp32 value, torch op on the widened CPU tensor)"""
    rule = int(rng.integers(0, 4))
    if rule == 0:
        return _native.SCALE_NONE, 1.0, lambda t: t
    if rule == 1:
        s = float(2.0 ** int(rng.integers(-3, 20)))
        return _native.SCALE_DIVIDE, s, lambda t: t.div_(s)
    if rule == 2:
        s = float(np.float32(rng.uniform(0.3, 5000.0)))
        return _native.SCALE_DIVIDE, s, lambda t: t.div_(s)
    f = float(np.float32(rng.uniform(0.01, 1.5)))
    return _native.SCALE_MULTIPLY, f, lambda t: t.mul_(f)


def _scan(tab, dtype, begin, end, ob, oe, mode, value, flat):
    lib = _native.load()
    nb = _native.stats_blocks()
    nt = _native.scan_tiles(end - begin)
    ps = torch.full((nb,), float("nan"), dtype=torch.float64, device=DEV)
    pf = torch.full((nb,), -1, dtype=torch.int32, device=DEV)
    ts = torch.full((nt + 1,), float("nan"), dtype=torch.float64, device=DEV)
    tf = torch.full((nt + 1,), -1, dtype=torch.int32, device=DEV)
    rc = lib.ms_grad_stats(tab.ptr, tab.nseg, _native.ms_dtype(dtype), begin, end, ob, oe, mode,
                           value, flat.data_ptr() if flat is not None else None, ts.data_ptr(),
                           tf.data_ptr(), nt, ps.data_ptr(), pf.data_ptr(), nb, stream())
    _native.check(rc, "ms_grad_stats")
    torch.cuda.synchronize()
    ts, tf = ts.cpu().numpy(), tf.cpu().numpy()
    assert np.isnan(ts[nt]) and tf[nt] == -1, "K1 wrote past its tile slots"
    return ps.cpu().numpy(), pf.cpu().numpy(), ts[:nt], tf[:nt]


@pytest.mark.parametrize("seed", range(48))
def test_k1_random_layouts(seed):
    rng, dtype, numels, host, missing, misaligned = _case(seed)
    dev = _device(host, missing, misaligned, dtype)
    lay = layout_for(numels)
    n = lay.numel_padded
    # the scanned range: the whole space, or a piece starting / ending inside
    # parameters; the owned range inside it
    if seed % 3 == 0:
        begin, end = 0, n
    else:
        begin = int(rng.integers(0, max(1, n // 2)))
        end = int(rng.integers(begin + 1, n + 1))
    ob = int(rng.integers(begin, end + 1)) if seed % 5 == 1 else begin
    oe = int(rng.integers(ob, end + 1)) if seed % 5 == 1 else end
    mode, value, op = _scaling(rng)
    tab = Table(lay, begin, end, [store(g, off) for g, off in zip(dev, lay.offsets)],
                [None] * len(numels))
    flat = torch.full((end - begin,), float("nan"), device=DEV)
    with_flat = _scan(tab, dtype, begin, end, ob, oe, mode, value, flat)
    without = _scan(tab, dtype, begin, end, ob, oe, mode, value, None)
    for a, b in zip(with_flat, without):
        np.testing.assert_array_equal(a.view(np.uint8), b.view(np.uint8))
    ps, pf, ts, tf = without

    # the oracle: widen (missing gradients are zeros), scale, over [begin, end)
    full = torch.zeros(n, dtype=torch.float32)
    raw_bad = np.zeros(n, dtype=bool)
    for x, miss, off in zip(host, missing, lay.offsets):
        if miss:
            continue
        w = x.float()
        full[off:off + x.numel()] = w
        raw_bad[off:off + x.numel()] = ~torch.isfinite(w).numpy()
    want = op(full[begin:end].clone())
    # bit for bit; NaNs as NaNs (their payloads after widening are not pinned)
    got = flat.cpu()
    nan = torch.isnan(want)
    np.testing.assert_array_equal(torch.isnan(got).numpy(), nan.numpy())
    np.testing.assert_array_equal(bits(got[~nan]), bits(want[~nan]))

    nt = ts.size
    assert nt == -(-(end - begin) // TILE)
    owned = want.numpy().astype(np.float64)
    owned[:ob - begin] = 0.0
    owned[oe - begin:] = 0.0
    bad = raw_bad[begin:end]
    for t in range(nt):
        a, b = t * TILE, min((t + 1) * TILE, end - begin)
        assert bool(tf[t]) == bool(bad[a:b].any()), t
        if not bad[a:b].any():
            exact = recipe.sumsq_f64(owned[a:b].astype(np.float32))
            assert abs(ts[t] - exact) <= 1e-12 * exact, t
    nblk = ps.size
    edges = np.arange(nblk + 1, dtype=np.int64) * nt // nblk
    for j in range(nblk):
        lo, hi = edges[j], edges[j + 1]
        assert bool(pf[j]) == bool(tf[lo:hi].any()), j
        if not tf[lo:hi].any():
            want_j = ts[lo:hi].sum()
            assert abs(ps[j] - want_j) <= 1e-12 * abs(want_j), j
