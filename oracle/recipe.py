"""numpy restatement of the HIP kernels' per-element arithmetic.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The kernels round exactly where minispeed's torch op sequence rounds
(optim/adam.py:82-91, flat.py:247, flat.py:255-257); on the CPU, torch
implements those ops as (probed on this torch build, no reference code run):

    add_(t, alpha)        fma(t, fp32(alpha), self)
    mul_(s)               self * fp32(s)
    addcmul_(a, b, value) fma(fp32(value) * a, b, self)
    addcdiv_(a, b, value) self + (fp32(value) * a) / b
    t / s                 IEEE division by fp32(s)
    sqrt                  MKL: correctly rounded except on ~0.6% of inputs

This module computes the same expression with numpy float32 ops, an exact
fp32 fused multiply-add and numpy's correctly rounded sqrt.  It is the
bit-exact expectation for the GPU kernels; against ``oracle.boundary`` it
differs only through the sqrt.  ``adamw_f64`` is the same update carried in
float64, the yardstick for ulp-error bounds.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def f32(x) -> np.float32:
    return np.float32(x)


def fma32(a, b, c) -> np.ndarray:
    """Exact fp32 fma(a, b, c) with round-to-nearest-even.

    a*b is exact in float64; t = a*b + c is rounded once in float64 and its
    rounding error e recovered exactly (TwoSum).  The final float32 rounding
    of t can only be wrong when t sits exactly on a float32 midpoint while
    e != 0; that case is resolved toward the sign of e.
    """
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    c = np.asarray(c, dtype=np.float32)
    p = a.astype(np.float64) * b.astype(np.float64)
    c64 = c.astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        t = p + c64
        bp = t - c64
        e = (p - bp) + (c64 - (t - bp))
        r = t.astype(np.float32)
        r64 = r.astype(np.float64)
        up = np.nextafter(r, np.float32(np.inf))
        dn = np.nextafter(r, np.float32(-np.inf))
        mid_up = (r64 + up.astype(np.float64)) * 0.5
        mid_dn = (r64 + dn.astype(np.float64)) * 0.5
        finite = np.isfinite(t) & np.isfinite(e)
        fix_up = finite & (t == mid_up) & (e > 0)
        fix_dn = finite & (t == mid_dn) & (e < 0)
    r = np.where(fix_up, up, r)
    r = np.where(fix_dn, dn, r)
    return r.astype(np.float32)


def adamw_step(p, m, v, g, *, lr, betas, eps, wd, step, grad_scale=1.0, unscale=False,
               clip_coef=None):
    """One element-wise AdamW update in the kernels' rounding order.

    ``g`` is the widened fp32 gradient (before unscale); ``clip_coef`` is the
    fp32 clip coefficient or None.  Returns new (p, m, v) as float32.
    """
    b1, b2 = float(betas[0]), float(betas[1])
    g = np.asarray(g, dtype=F32)
    p = np.asarray(p, dtype=F32).copy()
    m = np.asarray(m, dtype=F32)
    v = np.asarray(v, dtype=F32)
    if unscale:
        g = g / f32(grad_scale)
    if clip_coef is not None:
        g = g * f32(clip_coef)
    if wd != 0.0:
        p = fma32(p, f32(-lr * wd), p)
    m = fma32(g, f32(1.0 - b1), m * f32(b1))
    v = fma32(f32(1.0 - b2) * g, g, v * f32(b2))
    den = np.sqrt(v / f32(1.0 - b2 ** step)) + f32(eps)
    p = p + (f32(-lr) * (m / f32(1.0 - b1 ** step))) / den
    return p.astype(F32), m.astype(F32), v.astype(F32)


def adamw_f64(p, m, v, g, *, lr, betas, eps, wd, step, clip_coef=None):
    """The same update in float64 (g already unscaled)."""
    b1, b2 = float(betas[0]), float(betas[1])
    g = np.asarray(g, dtype=np.float64)
    if clip_coef is not None:
        g = g * float(clip_coef)
    p = np.asarray(p, dtype=np.float64) * (1.0 - lr * wd)
    m = np.asarray(m, dtype=np.float64) * b1 + (1.0 - b1) * g
    v = np.asarray(v, dtype=np.float64) * b2 + (1.0 - b2) * g * g
    den = np.sqrt(v / (1.0 - b2 ** step)) + eps
    p = p - lr * (m / (1.0 - b1 ** step)) / den
    return p, m, v


def ulp_distance(a, b) -> np.ndarray:
    """|a - b| in units of fp32 spacing, via the ordered integer map."""
    ai = np.asarray(a, dtype=np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, dtype=np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7FFFFFFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFFFFFF), bi)
    return np.abs(ai - bi)


def sumsq_f64(values) -> float:
    """Exactly-squared, float64-accumulated sum of squares."""
    x = np.asarray(values, dtype=np.float64)
    return float(np.dot(x, x))


def clip_coef(norm32: float, max_norm):
    """(applied, coef64, coef32) of stage_1_and_2.py:123-126 + flat.py:252."""
    if max_norm is None or not (float(norm32) > max_norm):
        return False, 1.0, 1.0
    coef = max_norm / (float(norm32) + 1e-6)
    return coef != 1.0, coef, float(np.float32(coef))
