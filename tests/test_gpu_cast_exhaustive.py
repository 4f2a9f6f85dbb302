"""fp32 -> fp16 / bf16 narrowing on every one of the 2^32 fp32 bit patterns.

The model copy the boundary writes is torch's fp32 -> param-dtype ``copy_``
(flat.py:133-154, stage_3.py:79-84): round to nearest even, overflow to
+-inf, subnormals kept.  K4 (``ms_cast_to_model``) and K3's model-copy
store (``ms_fused_adamw`` with lr = 0, weight decay 0 and zero gradients,
which leaves every non-NaN master bit-for-bit unchanged) are run over all
2^32 patterns in chunks of 2^28 and compared with torch's CPU conversion of
the same bits.  NaN inputs must give a NaN of the target type; their
payload bits are not compared (torch's CPU fp32 -> bf16 conversion itself
gives 0xFFFF on its vectorised path and 0x7FC0 on its scalar one).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import DEV, Table, adamw_params, k3, k4, layout_for, scalars_device, store

pytestmark = pytest.mark.gpu

CHUNK = 1 << 28

# (exponent mask, mantissa mask) of the target type's NaN encodings, as int16
NAN_FIELDS = {torch.float16: (0x7C00, 0x03FF), torch.bfloat16: (0x7F80, 0x007F)}


def _is_nan16(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    exp, man = NAN_FIELDS[dtype]
    return ((x & exp) == exp) & ((x & man) != 0)


@pytest.mark.parametrize("mdtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_every_fp32_pattern_narrows_like_torch(mdtype):
    lay = layout_for([CHUNK])
    zeros_g = torch.zeros(CHUNK, dtype=mdtype, device=DEV)
    m = torch.zeros(CHUNK, device=DEV)
    v = torch.zeros(CHUNK, device=DEV)
    model = torch.empty(CHUNK, dtype=mdtype, device=DEV)
    tab = Table(lay, 0, CHUNK, [store(zeros_g, 0)], [store(model, 0)])
    hp = adamw_params(0.0, (0.9, 0.999), 1e-8, 0.0, 1)
    sc = scalars_device()
    checked = 0
    for start in range(0, 1 << 32, CHUNK):
        u = np.arange(CHUNK, dtype=np.uint32) + np.uint32(start)
        x_cpu = torch.from_numpy(u.view(np.float32))
        want = x_cpu.to(mdtype).view(torch.int16).to(DEV)
        x = x_cpu.to(DEV)
        xi = x.view(torch.int32)
        nan_in = (xi & 0x7FFFFFFF) > 0x7F800000

        for kernel in ("k4", "k3"):
            model.view(torch.int16).fill_(0x5555)
            if kernel == "k4":
                k4(tab, mdtype, x, 0, CHUNK)
            else:
                p = x.clone()
                m.zero_()
                v.zero_()
                k3(tab, mdtype, mdtype, 0, CHUNK, p, m, v, hp, sc)
                moved = ((p.view(torch.int32) != xi) & ~nan_in).sum().item()
                assert moved == 0, f"{kernel} changed {moved} masters in chunk {start:#x}"
                assert bool(torch.isnan(p[nan_in]).all())
            got = model.view(torch.int16)
            bad = ((got != want) & ~nan_in).sum().item()
            assert bad == 0, f"{kernel} {mdtype}: {bad} mismatches in chunk {start:#x}"
            nan_lost = (nan_in & ~_is_nan16(got, mdtype)).sum().item()
            assert nan_lost == 0, f"{kernel} {mdtype}: {nan_lost} NaN inputs not NaN"
        checked += CHUNK
        print(f"[cast] {mdtype} chunk {start:#010x} ok", flush=True)
    assert checked == 1 << 32
