"""CPU restatement (numpy fp32) of the reference's RMSNorm kernels — TEST INFRASTRUCTURE ONLY.

The checker of the HIP norm kernels (include/smel_norm.h); nothing in the product path imports it. Every function
follows the reference file:line it names (paths relative to the reference repository root): fp32 arithmetic with
the same rounding points to the 16-bit dtype (``dt`` = "bf16" or "fp16"), row sums in fp32. Inputs are fp32 arrays
holding values of the 16-bit dtype; outputs are fp32 arrays holding rounded 16-bit values (rstd stays fp32).

``torch_*`` restate the reference's torch code for the same ops (smel/layer_runner.py:110-138), the comparator the
reference's own tests use (tests/test_norm.py:35-98).

PINNED (tests/test_norm_oracle.py):
  rmsnorm_fwd ....... fp64 closed form x / sqrt(mean(x^2) + eps) * w' (within one rounding), the torch path
  rmsnorm_bwd ....... fp64 autograd of the closed-form forward (with and without the residual gradient ds),
                      the torch path's autograd
  add_rmsnorm_fwd ... s bit-equal to torch's 16-bit h + x; y against the fp64 closed form of the rounded s
  gated_fwd / _bwd .. the torch path and its autograd (reference tolerance 1e-3), fp64 autograd of the formula
"""
from __future__ import annotations

import numpy as np
import torch

from .intref import bf16_bits_to_f32, bf16_rne

F32 = np.float32


def rnd(v: np.ndarray, dt: str) -> np.ndarray:
    """Round fp32 values to the 16-bit dtype (nearest even) and back to fp32."""
    v = np.asarray(v, dtype=F32)
    if dt == "bf16":
        return bf16_bits_to_f32(bf16_rne(v)).reshape(v.shape)
    if dt == "fp16":
        return v.astype(np.float16).astype(F32)
    raise ValueError(dt)


def w_eff(w, n: int, w_mode: int) -> np.ndarray:
    """smel/norm.py:41-48: mode 0 no weight (1), 1 w, 2 1 + w."""
    if w_mode == 0:
        return np.ones(n, dtype=F32)
    w = np.asarray(w, dtype=F32)
    return (F32(1.0) + w).astype(F32) if w_mode == 2 else w


def _rstd(x: np.ndarray, eps: float) -> np.ndarray:
    n = x.shape[-1]
    ms = (x * x).sum(axis=-1, dtype=F32) / F32(n)
    return (F32(1.0) / np.sqrt(ms + F32(eps))).astype(F32)


def rmsnorm_fwd(x, w, eps, w_mode, dt="bf16"):
    """smel/norm.py:50-62: rstd = 1 / sqrt(sum(x^2) / n + eps), y = x * rstd * w' -> dt."""
    x = np.asarray(x, dtype=F32)
    r = _rstd(x, eps)
    y = x * r[..., None] * w_eff(w, x.shape[-1], w_mode)
    return rnd(y, dt), r


def rmsnorm_bwd(dy, x, w, w_mode, rstd, ds=None, dt="bf16"):
    """smel/norm.py:64-82: xhat = x rstd, g = dy w', c = sum(g xhat) / n, dx = rstd (g - xhat c) (+ ds) -> dt."""
    dy, x = np.asarray(dy, dtype=F32), np.asarray(x, dtype=F32)
    n = x.shape[-1]
    r = np.asarray(rstd, dtype=F32)[..., None]
    xhat = x * r
    g = dy * w_eff(w, n, w_mode)
    c = (g * xhat).sum(axis=-1, dtype=F32)[..., None] / F32(n)
    dx = r * (g - xhat * c)
    if ds is not None:
        dx = dx + np.asarray(ds, dtype=F32)
    return rnd(dx, dt)


def add_rmsnorm_fwd(h, x, w, eps, w_mode, dt="bf16"):
    """smel/norm.py:84-100: s = (h + x) -> dt, stored; y = s rstd(s) w' -> dt."""
    s = rnd(np.asarray(h, dtype=F32) + np.asarray(x, dtype=F32), dt)
    y, r = rmsnorm_fwd(s, w, eps, w_mode, dt)
    return s, y, r


def _sigmoid(z):
    return (F32(1.0) / (F32(1.0) + np.exp(-z))).astype(F32)


def gated_fwd(x, z, w, eps, dt="bf16"):
    """smel/norm.py:102-119: n = (x rstd) -> dt, y = (w n) -> dt, out = y silu(z) -> dt."""
    x, z, w = (np.asarray(a, dtype=F32) for a in (x, z, w))
    r = _rstd(x, eps)
    nn = rnd(x * r[..., None], dt)
    y = rnd(w * nn, dt)
    return rnd(y * (z * _sigmoid(z)), dt), r


def gated_bwd(do, x, z, w, rstd, dt="bf16"):
    """smel/norm.py:121-145: dz = do y sg (1 + z (1 - sg)); dy = (do silu(z)) -> dt; dn = (dy w) -> dt;
    dx = rstd (dn - xhat sum(dn xhat) / n)."""
    do, x, z, w = (np.asarray(a, dtype=F32) for a in (do, x, z, w))
    n = x.shape[-1]
    r = np.asarray(rstd, dtype=F32)[..., None]
    xhat = x * r
    y = rnd(w * rnd(xhat, dt), dt)
    sg = _sigmoid(z)
    dz = do * y * (sg * (F32(1.0) + z * (F32(1.0) - sg)))
    dyv = rnd(do * (z * sg), dt)
    dn = rnd(dyv * w, dt)
    c = (dn * xhat).sum(axis=-1, dtype=F32)[..., None] / F32(n)
    dx = r * (dn - xhat * c)
    return rnd(dx, dt), rnd(dz, dt)


# ------------------------------------------------------------------ the reference's torch code (comparator)


def torch_rmsnorm(x: torch.Tensor, w, eps, plus_one=True):
    """smel/layer_runner.py:110-121 (torch branch)."""
    xf = x.float()
    if plus_one:
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
        return (xf * (1.0 + w.float())).type_as(x)
    xf = xf * torch.pow(xf.pow(2).mean(-1, keepdim=True) + eps, -0.5)
    return (xf if w is None else xf * w.float()).type_as(x)


def torch_add_rmsnorm(h, x, w, eps, plus_one=True):
    """smel/layer_runner.py:124-129 (torch branch)."""
    s = h + x
    return s, torch_rmsnorm(s, w, eps, plus_one)


def torch_gated_rmsnorm(x, z, w, eps):
    """smel/layer_runner.py:132-138 (torch branch)."""
    dt = x.dtype
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    y = w * xf.to(dt)
    return (y * torch.nn.functional.silu(z.float())).to(dt)
