"""RMSNorm family of the frozen layers around the MoE block, on the HIP kernels of libsmel_moe.so
(include/smel_norm.h): one launch forward, one backward.

  rmsnorm(x, w, eps, plus_one)          y = x * rstd * (1 + w) (Qwen3.5/3.6), x * rstd * w (Gemma 4), x * rstd (w None)
  add_rmsnorm(h, x, w, eps, plus_one)   s = h + x (the residual add), y = rmsnorm(s)
  gated_rmsnorm(x, z, w, eps)           y = w * norm(x) * silu(z)  (output norm of Gated DeltaNet)

The API is the reference's smel/norm.py:252-275 (``supported``, ``ENABLED``, ``MAX_COLS`` and the three functions,
same arguments and return values). The norm weights are frozen, so backward gives dx (and dz) only, as there.
fp32 math with the reference's rounding points (the residual sum rounded to the stream's dtype, the gated norm's
``n`` and ``w n`` rounded); saved for backward: the input and one fp32 rstd per row:

    xhat = x * rstd,  g = dy * w',  dx = rstd * (g - xhat * mean(g * xhat))     (w' = 1 + w, w or 1)

There is no fallback: without the library every call raises. ``supported`` answers the same question as the
reference's (16-bit rows on the GPU, frozen contiguous weights of the rows' dtype, at most MAX_COLS columns), so a
caller that routes other cases to its own torch code keeps doing so.
"""
from __future__ import annotations

import torch

from . import _lib

MAX_COLS = 16384
ENABLED = True   # callers switch the kernels off to compare with their torch code

_DTYPES = {torch.bfloat16: 0, torch.float16: 1}


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype not in _DTYPES:
        raise ValueError(f"smel norms take bf16 or fp16 rows, got {t.dtype}")
    return _DTYPES[t.dtype]


def _check_weight(w, x):
    if w is not None and (w.dtype != x.dtype or w.numel() != x.shape[-1] or not w.is_contiguous()):
        raise ValueError(f"norm weight must be a contiguous [{x.shape[-1]}] tensor of {x.dtype}")


def _rows(x: torch.Tensor):
    """x as [rows, n_cols] with unit column stride and its row stride; a strided view (rows further apart than
    n_cols, e.g. a chunk of a wider projection) is used in place (smel/norm.py:148-154)."""
    n_cols = x.shape[-1]
    x2 = x.reshape(-1, n_cols)
    if x2.stride(-1) != 1 or (x2.shape[0] > 1 and x2.stride(0) < n_cols):
        x2 = x2.contiguous()
    return x2, (x2.stride(0) if x2.shape[0] > 1 else n_cols)


class _RMSNorm(torch.autograd.Function):
    """smel/norm.py:157-183."""

    @staticmethod
    def forward(ctx, x, w, eps, w_mode):
        _lib.require_device(x, w)
        _check_weight(w, x)
        x2, xs = _rows(x)
        rows, n = x2.shape
        y = torch.empty(x.shape, device=x.device, dtype=x.dtype)
        rstd = torch.empty(rows, device=x.device, dtype=torch.float32)
        _lib.call("smel_rmsnorm_fwd", _lib.ptr(x2), rows, n, xs, _lib.ptr(w), w_mode, float(eps), _dtype_code(x),
                  _lib.ptr(y), _lib.ptr(rstd), _lib.stream())
        ctx.save_for_backward(x2, w, rstd)
        ctx.shape, ctx.xs, ctx.w_mode = x.shape, xs, w_mode
        return y

    @staticmethod
    def backward(ctx, dy):
        x2, w, rstd = ctx.saved_tensors
        rows, n = x2.shape
        dy2 = dy.reshape(rows, n).contiguous()
        dx = torch.empty(ctx.shape, device=dy.device, dtype=x2.dtype)
        _lib.call("smel_rmsnorm_bwd", _lib.ptr(dy2), _lib.ptr(x2), rows, n, ctx.xs, _lib.ptr(w), ctx.w_mode,
                  _lib.ptr(rstd), None, _dtype_code(x2), _lib.ptr(dx), _lib.stream())
        return dx, None, None, None


class _AddRMSNorm(torch.autograd.Function):
    """smel/norm.py:186-219: both inputs get the same gradient, the norm's dx plus the gradient of s's other use
    (added in fp32 before the one rounding)."""

    @staticmethod
    def forward(ctx, h, x, w, eps, w_mode):
        _lib.require_device(h, x, w)
        _check_weight(w, h)
        n = h.shape[-1]
        h2, x2 = h.reshape(-1, n).contiguous(), x.reshape(-1, n).contiguous()
        rows = h2.shape[0]
        s = torch.empty(h.shape, device=h.device, dtype=h.dtype)
        y = torch.empty(h.shape, device=h.device, dtype=h.dtype)
        rstd = torch.empty(rows, device=h.device, dtype=torch.float32)
        _lib.call("smel_add_rmsnorm_fwd", _lib.ptr(h2), _lib.ptr(x2), rows, n, _lib.ptr(w), w_mode, float(eps),
                  _dtype_code(h), _lib.ptr(s), _lib.ptr(y), _lib.ptr(rstd), _lib.stream())
        ctx.save_for_backward(s, w, rstd)
        ctx.w_mode = w_mode
        ctx.set_materialize_grads(False)
        return s, y

    @staticmethod
    def backward(ctx, ds, dy):
        s, w, rstd = ctx.saved_tensors
        if dy is None:
            return ds, ds, None, None, None
        n = s.shape[-1]
        s2 = s.reshape(-1, n)
        rows = s2.shape[0]
        dy2 = dy.reshape(rows, n).contiguous()
        ds2 = ds.reshape(rows, n).contiguous() if ds is not None else None
        d = torch.empty(s.shape, device=s.device, dtype=s.dtype)
        _lib.call("smel_rmsnorm_bwd", _lib.ptr(dy2), _lib.ptr(s2), rows, n, n, _lib.ptr(w), ctx.w_mode,
                  _lib.ptr(rstd), _lib.ptr(ds2), _dtype_code(s), _lib.ptr(d), _lib.stream())
        return d, d, None, None, None


class _GatedRMSNorm(torch.autograd.Function):
    """smel/norm.py:222-249."""

    @staticmethod
    def forward(ctx, x, z, w, eps):
        _lib.require_device(x, z, w)
        _check_weight(w, x)
        n = x.shape[-1]
        x2, z2 = x.reshape(-1, n).contiguous(), z.reshape(-1, n).contiguous()
        rows = x2.shape[0]
        y = torch.empty(x.shape, device=x.device, dtype=x.dtype)
        rstd = torch.empty(rows, device=x.device, dtype=torch.float32)
        _lib.call("smel_gated_rmsnorm_fwd", _lib.ptr(x2), _lib.ptr(z2), rows, n, _lib.ptr(w), float(eps),
                  _dtype_code(x), _lib.ptr(y), _lib.ptr(rstd), _lib.stream())
        ctx.save_for_backward(x2, z2, w, rstd)
        ctx.shapes = (x.shape, z.shape)
        return y

    @staticmethod
    def backward(ctx, dout):
        x2, z2, w, rstd = ctx.saved_tensors
        rows, n = x2.shape
        do2 = dout.reshape(rows, n).contiguous()
        dx = torch.empty(ctx.shapes[0], device=dout.device, dtype=x2.dtype)
        dz = torch.empty(ctx.shapes[1], device=dout.device, dtype=z2.dtype)
        _lib.call("smel_gated_rmsnorm_bwd", _lib.ptr(do2), _lib.ptr(x2), _lib.ptr(z2), rows, n, _lib.ptr(w),
                  _lib.ptr(rstd), _dtype_code(x2), _lib.ptr(dx), _lib.ptr(dz), _lib.stream())
        return dx, dz, None, None


def supported(x, *weights):
    """The kernels apply to a GPU bf16/fp16 input whose norm weights are frozen, contiguous, of the input's dtype and
    shape [n_cols], with n_cols <= MAX_COLS (smel/norm.py:252-259)."""
    if not (ENABLED and x.is_cuda and x.dtype in _DTYPES):
        return False
    if x.shape[-1] > MAX_COLS:
        return False
    return all(w is None or (w.dtype == x.dtype and not w.requires_grad and w.is_contiguous()
                             and tuple(w.shape) == (x.shape[-1],)) for w in weights)


def rmsnorm(x, w, eps, plus_one):
    return _RMSNorm.apply(x, w, eps, 0 if w is None else (2 if plus_one else 1))


def add_rmsnorm(h, x, w, eps, plus_one):
    """(h + x, rmsnorm(h + x)): the residual add and the norm after it."""
    return _AddRMSNorm.apply(h, x, w, eps, 2 if plus_one else 1)


def gated_rmsnorm(x, z, w, eps):
    return _GatedRMSNorm.apply(x, z, w, eps)
