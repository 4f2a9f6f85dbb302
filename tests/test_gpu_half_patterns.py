"""K1 over every fp16 and bf16 bit pattern: the inf/nan flag, the widening
and unscale, and the sum of squares.

The reference tests ``torch.isfinite`` on the widened, pre-unscale flat
gradient (precision.py:79-92, engine.py:275) and then divides it by the
loss scale (flat.py:243-247).  K1's vector path decides finiteness with a
packed test on 32-bit words (two halves at a time), its scalar path (segment
edges, misaligned storage) one element at a time; both are run here on all
65,536 patterns of each half type.

Layout of one launch, with B = ms_stats_min_chunk() (65536): n = (16 +
#non-finite) x B elements, so K1 runs one block per B-element range and
reports one flag per block.  Blocks 0-15
hold every finite pattern, eight times over at the eight positions of a
16-byte vector (block 2s and 2s+1 hold the list rotated by s); block 16+j
holds non-finite pattern j alone among zeros, at position 8j + (j mod 8) so
that each one lands in every lane slot somewhere.  Flags must be exactly
"block >= 16"; the materialized flat gradient of blocks 0-15 must equal
torch's CPU ``x.float().div_(scale)`` bit for bit, and each finite block's
fp64 partial must equal the exact sum of squares to 1e-12.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import recipe
from minispeed_amd import _native
from tests.helpers import DEV, Table, bits, k1, layout_for, store

pytestmark = pytest.mark.gpu

FINITE_BLOCKS = 16
EXP_FIELD = {torch.float16: 0x7C00, torch.bfloat16: 0x7F80}


def _patterns(dtype):
    allp = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    e = EXP_FIELD[dtype]
    nonfinite = allp[(allp & e) == e]
    finite = allp[(allp & e) != e]
    return finite, nonfinite


def _host_buffer(dtype, block):
    finite, nonfinite = _patterns(dtype)
    nblk = FINITE_BLOCKS + nonfinite.size
    assert finite.size <= 2 * block and 8 * nonfinite.size <= block
    buf = np.zeros(nblk * block, dtype=np.uint16)
    pair = np.zeros(2 * block, dtype=np.uint16)
    pair[:finite.size] = finite
    for s in range(8):
        buf[2 * s * block:(2 * s + 2) * block] = np.roll(pair, s)
    for j, pat in enumerate(nonfinite):
        buf[(FINITE_BLOCKS + j) * block + 8 * j + j % 8] = pat
    return buf, nblk


@pytest.mark.parametrize("scale", [1.0, 65536.0, 1000.0])
@pytest.mark.parametrize("aligned", [True, False], ids=["vector", "scalar"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_every_half_pattern(dtype, aligned, scale):
    block = _native.stats_min_chunk()
    raw, nblk = _host_buffer(dtype, block)
    assert nblk <= _native.stats_blocks()
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
    psum, pflag = k1(tab, dtype, 0, n, 0, n, scale=scale, flat=flat)

    # one flag per block of the nblk-block grid; the slots after it read 0
    want_flag = np.zeros(pflag.size, dtype=bool)
    want_flag[FINITE_BLOCKS:nblk] = True
    np.testing.assert_array_equal(pflag != 0, want_flag)
    assert not psum[nblk:].any()

    fin = FINITE_BLOCKS * block
    want = host[:fin].float().div_(scale)
    got = flat[:fin].cpu()
    np.testing.assert_array_equal(bits(got), bits(want))
    for b in range(FINITE_BLOCKS):
        exact = recipe.sumsq_f64(want[b * block:(b + 1) * block].numpy())
        assert abs(psum[b] - exact) <= 1e-12 * exact, b

    # the non-finite blocks: the pattern itself widens to the same inf/nan
    nf = flat[fin:].cpu().numpy().reshape(-1, block)
    src = host[fin:].float().div_(scale).numpy().reshape(-1, block)
    for j in range(nf.shape[0]):
        k = 8 * j + j % 8
        if np.isnan(src[j, k]):
            assert np.isnan(nf[j, k]), j
        else:
            assert nf[j, k] == src[j, k], j
