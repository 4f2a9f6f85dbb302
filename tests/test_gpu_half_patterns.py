"""K1 over every fp16 and bf16 bit pattern: the inf/nan flag, the widening
and unscale, and the sum of squares.

The reference tests ``torch.isfinite`` on the widened, pre-unscale flat
gradient (precision.py:79-92, engine.py:275) and then divides it by the
loss scale (flat.py:243-247).  K1's vector path decides finiteness with a
packed test on 32-bit words (two halves at a time), its scalar path (segment
edges, misaligned storage) one element at a time; both are run here on all
65,536 patterns of each half type.

Layout of one launch, in K1 tiles of T = MS_SCAN_TILE (2048) elements:
eight copies of the list of finite patterns, copy s rotated by s, each
copy zero-padded to whole tiles, so every finite pattern sits at all eight
positions of a 16-byte vector; then one tile per non-finite pattern j,
alone among zeros at position 8 (j mod 256) + (j mod 8), so that the
patterns land in every unit slot and every position of a unit.  Tile flags
must be exactly "tile >= finite tiles" and the partial slots' flags the OR
over the tiles each slot folds; the materialized flat gradient of the finite
tiles must equal torch's CPU ``x.float().div_(scale)`` bit for bit, each
finite tile's fp64 sum must equal the exact sum of squares to 1e-12 and
each partial slot the sum of its tiles.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from minispeed_amd import _native
from oracle import recipe
from tests.helpers import DEV, Table, bits, k1, layout_for, store

pytestmark = pytest.mark.gpu

TILE = _native.SCAN_TILE
EXP_FIELD = {torch.float16: 0x7C00, torch.bfloat16: 0x7F80}


def _patterns(dtype):
    allp = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    e = EXP_FIELD[dtype]
    nonfinite = allp[(allp & e) == e]
    finite = allp[(allp & e) != e]
    return finite, nonfinite


def _host_buffer(dtype):
    """(buffer, finite tiles, all tiles)"""
    finite, nonfinite = _patterns(dtype)
    per_copy = -(-finite.size // TILE)
    fin_tiles = 8 * per_copy
    ntiles = fin_tiles + nonfinite.size
    buf = np.zeros(ntiles * TILE, dtype=np.uint16)
    copy = np.zeros(per_copy * TILE, dtype=np.uint16)
    copy[:finite.size] = finite
    for s in range(8):
        buf[s * copy.size:(s + 1) * copy.size] = np.roll(copy, s)
    for j, pat in enumerate(nonfinite):
        buf[(fin_tiles + j) * TILE + 8 * (j % 256) + j % 8] = pat
    return buf, fin_tiles, ntiles


@pytest.mark.parametrize("scale", [1.0, 65536.0, 1000.0])
@pytest.mark.parametrize("aligned", [True, False], ids=["vector", "scalar"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_every_half_pattern(dtype, aligned, scale):
    raw, fin_tiles, ntiles = _host_buffer(dtype)
    n = raw.size
    host = torch.from_numpy(raw.view(np.int16)).view(dtype)
    if aligned:
        g = host.to(DEV)
    else:
        # storage offset of one element: 2-byte aligned, so every element
        # of the segment takes the per-element path
        base = torch.zeros(n + 1, dtype=dtype, device=DEV)
        base[1:].copy_(host.to(DEV))
        g = base[1:]
        assert g.data_ptr() % 16 != 0
    lay = layout_for([n])
    tab = Table(lay, 0, n, [store(g, 0)], [None])
    flat = torch.full((n,), float("nan"), device=DEV)
    psum, pflag, tsum, tflag = k1(tab, dtype, 0, n, 0, n, scale=scale, flat=flat, tiles=True)

    assert tsum.size == ntiles
    np.testing.assert_array_equal(tflag != 0, np.arange(ntiles) >= fin_tiles)
    # the fold: slot j covers tiles [j*nt/nblk, (j+1)*nt/nblk)
    nblk = psum.size
    edges = np.arange(nblk + 1, dtype=np.int64) * ntiles // nblk
    want_flag = np.array([(tflag[a:b] != 0).any() for a, b in zip(edges[:-1], edges[1:])])
    np.testing.assert_array_equal(pflag != 0, want_flag)
    fin_sum = np.where(np.arange(ntiles) < fin_tiles, tsum, 0.0)
    for j in np.flatnonzero(edges[1:] <= fin_tiles):
        want = fin_sum[edges[j]:edges[j + 1]].sum()
        assert abs(psum[j] - want) <= 1e-12 * abs(want), j

    fin = fin_tiles * TILE
    want = host[:fin].float().div_(scale)
    got = flat[:fin].cpu()
    np.testing.assert_array_equal(bits(got), bits(want))
    for t in range(fin_tiles):
        exact = recipe.sumsq_f64(want[t * TILE:(t + 1) * TILE].numpy())
        assert abs(tsum[t] - exact) <= 1e-12 * exact, t

    # the non-finite tiles: the pattern itself widens to the same inf/nan
    nf = flat[fin:].cpu().numpy().reshape(-1, TILE)
    src = host[fin:].float().div_(scale).numpy().reshape(-1, TILE)
    for j in range(nf.shape[0]):
        k = 8 * (j % 256) + j % 8
        if np.isnan(src[j, k]):
            assert np.isnan(nf[j, k]), j
        else:
            assert nf[j, k] == src[j, k], j
