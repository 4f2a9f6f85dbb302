"""Pins of oracle.recipe, the bit-exact expectation for the HIP kernels.

* fma32 against exact rational arithmetic, including a constructed case
  where rounding through float64 first would give the wrong fp32 result;
* the recipe equals the torch restatement (oracle.boundary.adam_update) bit
  for bit once it uses torch's own sqrt, so the two differ only through
  MKL's sqrt rounding;
* the recipe against the textbook torch.optim.AdamW (an independent
  implementation of the same update: a dropped term or sign fails) and
  against a float64 evaluation (rounding-error bound);
* the clip coefficient and sum-of-squares helpers against closed forms.
"""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import boundary as ob
from oracle import recipe


def _rn_f32(x: Fraction) -> np.float32:
    f = np.float32(float(x))
    best = None
    for c in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
        d = abs(Fraction(float(c)) - x)
        key = (d, int(np.array(c, dtype=np.float32).view(np.int32)) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return best[1]


def test_fma32_is_exactly_rounded():
    rng = np.random.default_rng(0)
    a = (rng.normal(size=3000) * np.exp(rng.uniform(-20, 20, 3000))).astype(np.float32)
    b = rng.normal(size=3000).astype(np.float32)
    c = (rng.normal(size=3000) * np.exp(rng.uniform(-20, 20, 3000))).astype(np.float32)
    got = recipe.fma32(a, b, c)
    for i in range(3000):
        want = _rn_f32(Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i])))
        assert got[i] == want, i


def test_fma32_resolves_float64_double_rounding():
    # a*b = 2^-24 - 2^-64, c = 1 + 2^-23: the exact sum lies just below the
    # midpoint between 1+2^-23 and 1+2^-22; float64 rounds it onto the
    # midpoint and a second rounding would pick 1+2^-22.
    a = np.float32(2.0 ** -12 * (1 + 2.0 ** -20))
    b = np.float32(2.0 ** -12 * (1 - 2.0 ** -20))
    c = np.float32(1 + 2.0 ** -23)
    naive = np.float32(np.float64(a) * np.float64(b) + np.float64(c))
    assert naive == np.float32(1 + 2.0 ** -22)
    assert recipe.fma32(a, b, c) == np.float32(1 + 2.0 ** -23)
    assert recipe.fma32(-a, -b, -c) == np.float32(-(1 + 2.0 ** -23))


@pytest.fixture
def torch_sqrt(monkeypatch):
    monkeypatch.setattr(recipe.np, "sqrt",
                        lambda x: torch.from_numpy(np.ascontiguousarray(x)).sqrt().numpy())


@pytest.mark.parametrize("wd,clip,scale", [(0.01, 0.37, 1.0), (0.0, None, 1.0), (0.1, None, 65536.0),
                                           (0.01, 0.9, 1000.0)])
def test_recipe_equals_torch_restatement_up_to_sqrt(torch_sqrt, wd, clip, scale):
    rng = np.random.default_rng(1)
    n = 200_000
    p = rng.normal(0, 0.02, n).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    for step in range(1, 5):
        raw = (rng.normal(0, 1e-3, n) * scale).astype(np.float16).astype(np.float32)
        tp, tm, tv = (torch.from_numpy(x.copy()) for x in (p, m, v))
        tg = torch.from_numpy(raw.copy())
        if scale != 1.0:
            tg.div_(scale)                                    # flat.py:247
        if clip is not None:
            tg.mul_(clip)                                     # flat.py:255
        ob.adam_update(tp, tg, tm, tv, 1e-3, (0.9, 0.999), 1e-8, wd, step)
        p, m, v = recipe.adamw_step(p, m, v, raw, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, wd=wd,
                                    step=step, grad_scale=scale, unscale=scale != 1.0,
                                    clip_coef=clip)
        for got, want in ((p, tp), (m, tm), (v, tv)):
            np.testing.assert_array_equal(got.view(np.int32), want.numpy().view(np.int32))


def test_recipe_and_torch_restatement_differ_only_slightly_with_real_sqrt():
    rng = np.random.default_rng(2)
    n = 500_000
    p = rng.normal(0, 0.02, n).astype(np.float32)
    m = rng.normal(0, 1e-3, n).astype(np.float32)
    v = (rng.random(n) * 1e-6).astype(np.float32)
    g = rng.normal(0, 1e-3, n).astype(np.float32)
    tp, tm, tv = (torch.from_numpy(x.copy()) for x in (p, m, v))
    ob.adam_update(tp, torch.from_numpy(g.copy()), tm, tv, 1e-3, (0.9, 0.999), 1e-8, 0.01, 7)
    rp, rm, rv = recipe.adamw_step(p, m, v, g, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, wd=0.01, step=7)
    np.testing.assert_array_equal(rm, tm.numpy())
    np.testing.assert_array_equal(rv, tv.numpy())
    differ = rp != tp.numpy()
    assert differ.mean() < 0.02
    scale = np.maximum(np.abs(p), np.abs(tp.numpy()))
    assert np.all(np.abs(rp.astype(np.float64) - tp.numpy()) <= 2 * np.spacing(scale))


def test_recipe_matches_textbook_adamw():
    """torch.optim.AdamW is an independent implementation of the same
    decoupled-decay update (minispeed's tests/test_engine.py:23-64 compares
    against it at rtol 1e-4)."""
    rng = np.random.default_rng(3)
    n = 50_000
    p0 = rng.normal(0, 0.02, n).astype(np.float32)
    param = torch.nn.Parameter(torch.from_numpy(p0.copy()))
    opt = torch.optim.AdamW([param], lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01,
                            foreach=False)
    p, m, v = p0, np.zeros(n, np.float32), np.zeros(n, np.float32)
    for step in range(1, 11):
        g = rng.normal(0, 1e-3, n).astype(np.float32)
        param.grad = torch.from_numpy(g.copy())
        opt.step()
        p, m, v = recipe.adamw_step(p, m, v, g, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, wd=0.01,
                                    step=step)
    st = opt.state[param]
    # torch.optim.AdamW rounds differently (lerp for exp_avg, sqrt of the bias
    # correction folded into the step size): compare at rtol 1e-5 with an
    # absolute floor of 1e-6 of each array's scale for elements near zero
    for mine, theirs in ((p, param.detach().numpy()), (m, st["exp_avg"].numpy()),
                         (v, st["exp_avg_sq"].numpy())):
        np.testing.assert_allclose(mine, theirs, rtol=1e-5, atol=1e-6 * np.abs(theirs).max())


def test_recipe_rounding_error_against_float64():
    rng = np.random.default_rng(4)
    n = 200_000
    p = rng.normal(0, 0.02, n).astype(np.float32)
    m = rng.normal(0, 1e-3, n).astype(np.float32)
    v = (rng.random(n) * 1e-6 + 1e-9).astype(np.float32)
    g = rng.normal(0, 1e-3, n).astype(np.float32)
    rp, rm, rv = recipe.adamw_step(p, m, v, g, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, wd=0.01,
                                   step=3, clip_coef=0.5)
    # the fp32 clip coefficient is part of the input
    ep, em, ev = recipe.adamw_f64(p, m, v, g * np.float32(0.5), lr=1e-3, betas=(0.9, 0.999),
                                  eps=1e-8, wd=0.01, step=3)
    # bounds in ulps of the largest operand of each update (cancellation
    # makes a bound relative to the result meaningless near zero)
    gc = np.abs(g * np.float32(0.5)).astype(np.float64)
    m_scale = np.maximum.reduce([np.abs(m), 0.1 * gc, np.abs(em)]).astype(np.float32)
    v_scale = np.maximum.reduce([v, 1e-3 * gc * gc, ev]).astype(np.float32)
    assert np.all(np.abs(rm - em) <= 2 * np.spacing(m_scale))
    assert np.all(np.abs(rv - ev) <= 3 * np.spacing(v_scale))
    upd = np.abs(ep - p)
    # eight rounded operations on the master path (constants included)
    assert np.all(np.abs(rp - ep) <= 8 * np.spacing(np.maximum(np.abs(p), upd).astype(np.float32)))


def test_clip_coef_and_sumsq_closed_forms():
    assert recipe.clip_coef(0.5, 1.0) == (False, 1.0, 1.0)
    assert recipe.clip_coef(1.0, 1.0) == (False, 1.0, 1.0)          # strict >
    applied, c64, c32 = recipe.clip_coef(np.float32(4.0), 1.0)
    assert applied and c64 == 1.0 / (4.0 + 1e-6) and c32 == float(np.float32(c64))
    assert recipe.clip_coef(3.0, None)[0] is False
    x = np.random.default_rng(5).normal(size=10_000).astype(np.float32)
    assert recipe.sumsq_f64(x) == pytest.approx(math.fsum(float(t) ** 2 for t in x), rel=1e-15)


def test_ulp_distance():
    one = np.float32(1.0)
    assert recipe.ulp_distance(one, np.nextafter(one, np.float32(2))) == 1
    assert recipe.ulp_distance(np.float32(-0.0), np.float32(0.0)) == 0
    assert recipe.ulp_distance(np.float32(-1e-45), np.float32(1e-45)) == 2


def test_master_step_check_accounts_for_every_element():
    """tests/helpers.py:master_step_within_ulps, the per-step master check of
    the GPU tests, on the CPU: the oracle's torch AdamW (CPU sqrt) as the
    reference side, the recipe (correctly rounded sqrt) in place of the GPU.
    It passes, and a one-ulp change of one GPU master, or the oracle run
    with another lr, makes it fail."""
    from tests.helpers import master_step_within_ulps

    rng = np.random.default_rng(11)
    n = 50_000
    p = rng.normal(0, 0.02, n).astype(np.float32)
    m = rng.normal(0, 1e-3, n).astype(np.float32)
    v = (rng.random(n) * 1e-6 + 1e-9).astype(np.float32)
    g = rng.normal(0, 1e-3, n).astype(np.float32)
    hp = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, wd=0.01, step=7)
    tp, tm, tv = (torch.from_numpy(x.copy()) for x in (p, m, v))
    ob.adam_update(tp, torch.from_numpy(g.copy()), tm, tv, hp["lr"], hp["betas"], hp["eps"],
                   hp["wd"], hp["step"])
    rp, rm, rv = recipe.adamw_step(p, m, v, g, **hp)
    assert np.array_equal(rm.view(np.int32), tm.numpy().view(np.int32))
    assert np.array_equal(rv.view(np.int32), tv.numpy().view(np.int32))
    ok, worst, nsq = master_step_within_ulps(p, rp, tp.numpy(), rm, rv, **hp)
    assert ok and worst <= 2.0 and nsq >= 0, (worst, nsq)
    # torch's sqrt differs from the correctly rounded one on some inputs
    q = rv / np.float32(1 - 0.999 ** 7)
    assert np.any(torch.from_numpy(q.copy()).sqrt().numpy() != np.sqrt(q))
    bad = rp.copy()
    k = int(np.argmax(np.abs(rp)))
    bad[k] = np.nextafter(bad[k], np.float32(np.inf))
    assert not master_step_within_ulps(p, bad, tp.numpy(), rm, rv, **hp)[0]
    assert not master_step_within_ulps(p, rp, tp.numpy(), rm, rv, **dict(hp, lr=1.1e-3))[0]
