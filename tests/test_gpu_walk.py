"""The C++ pointer walk that feeds the segment tables, on the GPU.

Its addresses must be exactly the tensors' own, and every gradient or
parameter it does not accept must go through the Python checks: a
non-contiguous gradient is copied, a wrong dtype or size raises.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

from minispeed_amd.flat import FlatParamGroup

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
SHAPES = [(7, 5), (3,), (6, 4), (1,), (129,), (2, 3)]


def _group(dtype=torch.float16):
    params = [nn.Parameter(torch.randn(*s, device=DEV).to(dtype)) for s in SHAPES]
    return params, FlatParamGroup(params, device=DEV, rank=0, world_size=1, zero_stage=1)


def test_addresses_are_the_tensors_own():
    params, g = _group()
    for k, p in enumerate(params):
        p.grad = None if k == 3 else torch.randn_like(p)
    ptrs, keep, gdt = g.grad_pointers()
    assert gdt is None
    assert ptrs.dtype == np.int64 and ptrs.shape == (len(params) + 1,) and ptrs[-1] == 0
    for k, p in enumerate(params):
        if p.grad is None:
            assert ptrs[k] == 0 and keep[k] is None
        else:
            assert ptrs[k] == p.grad.data_ptr() and keep[k] is p.grad
    mptrs = g.model_pointers()
    assert list(mptrs[:-1]) == [p.data_ptr() for p in params] and mptrs[-1] == 0


def test_non_contiguous_gradient_is_copied_and_the_rest_still_walked():
    params, g = _group()
    for p in params:
        p.grad = torch.randn_like(p)
    params[2].grad = torch.randn(4, 6, device=DEV, dtype=torch.float16).t()   # (6, 4) strided
    assert not params[2].grad.is_contiguous()
    ptrs, keep, gdt = g.grad_pointers()
    assert gdt is None
    assert keep[2].is_contiguous() and torch.equal(keep[2], params[2].grad)
    assert ptrs[2] == keep[2].data_ptr() != params[2].grad.data_ptr()
    for k in (0, 1, 3, 4, 5):
        assert ptrs[k] == params[k].grad.data_ptr() and keep[k] is params[k].grad


def test_gradient_of_another_dtype_widens_the_group():
    """minispeed's flatten copies any gradient dtype into the fp32 flat
    buffer (flat.py:209-212): one fp32 gradient in an fp16 group makes the
    walk widen every gradient of the group into one fp32 buffer."""
    params, g = _group()
    for k, p in enumerate(params):
        p.grad = None if k == 3 else torch.randn_like(p)
    if hasattr(params[4], "grad_dtype"):
        params[4].grad_dtype = None      # torch >= 2.10 checks .grad's dtype unless told not to
    params[4].grad = torch.randn(129, device=DEV)
    ptrs, keep, gdt = g.grad_pointers()
    assert gdt == 0                                    # MS_DTYPE_F32
    buf = keep[-1]
    assert buf.dtype == torch.float32 and buf.numel() == g.numel
    torch.cuda.synchronize()
    for k, p in enumerate(params):
        off, n = g.layout.offsets[k], g.layout.numels[k]
        if p.grad is None:
            assert ptrs[k] == 0
            continue
        assert ptrs[k] == buf.data_ptr() + 4 * off
        assert torch.equal(buf[off:off + n], p.grad.reshape(-1).float())
    if hasattr(params[5], "grad_dtype"):
        params[5].grad_dtype = None
    params[5].grad = torch.zeros(2, 3, device=DEV, dtype=torch.float64)
    with pytest.raises(TypeError, match="float64"):
        g.grad_pointers()


def test_gradient_of_another_size_raises():
    params, g = _group()
    for p in params:
        p.grad = torch.randn_like(p)
    params[1].data = torch.zeros(5, device=DEV, dtype=torch.float16)
    params[1].grad = torch.zeros(5, device=DEV, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="5 elements, expected 3"):
        g.grad_pointers()


def test_model_pointers_refuse_strided_or_mixed_parameters():
    params, g = _group()
    params[2].data = torch.zeros(4, 6, device=DEV, dtype=torch.float16).t()
    with pytest.raises(RuntimeError, match="contiguous"):
        g.model_pointers()
    params, g = _group()
    params[5].data = params[5].data.float()
    with pytest.raises(TypeError, match="share a dtype"):
        g.model_pointers()
