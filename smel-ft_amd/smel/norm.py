"""RMSNorm family of the frozen layers around the MoE block, on the HIP kernels of libsmel_moe.so
(include/smel_norm.h): one launch forward, one backward.

  rmsnorm(x, w, eps, plus_one)          y = x * rstd * (1 + w) (Qwen3.5/3.6), x * rstd * w (Gemma 4), x * rstd (w None)
  add_rmsnorm(h, x, w, eps, plus_one)   s = h + x (the residual add), y = rmsnorm(s)
  gated_rmsnorm(x, z, w, eps)           y = w * norm(x) * silu(z)  (output norm of Gated DeltaNet)

The API is the reference's smel/norm.py:252-275 (``supported``, ``ENABLED``, ``MAX_COLS`` and the three functions,
same arguments and return values). The norm weights are frozen, so backward gives dx (and dz) only, as there.
fp32 math with the reference's rounding points (the residual sum rounded to the stream's dtype, the gated norm's
``n`` and ``w n`` rounded); saved for backward: the rows the norm read and one fp32 rstd per row:

    xhat = x * rstd,  g = dy * w',  dx = rstd * (g - xhat * mean(g * xhat))     (w' = 1 + w, w or 1)

Structure: one autograd node (``_NormFn``) serves the three kinds; a kind is a forward launch and a backward launch
over [rows, n] operands. There is no fallback: without the library every call raises. ``supported`` answers the same
question as the reference's (16-bit rows on the GPU, frozen contiguous weights of the rows' dtype, at most MAX_COLS
columns), so a caller that routes other cases to its own torch code keeps doing so.
"""
from __future__ import annotations

import torch

from . import _lib

MAX_COLS = 16384
ENABLED = True   # callers switch the kernels off to compare with their torch code

_DTYPES = {torch.bfloat16: 0, torch.float16: 1}
_RMS, _ADD, _GATED = "rms", "add", "gated"


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype not in _DTYPES:
        raise ValueError(f"smel norms take bf16 or fp16 rows, got {t.dtype}")
    return _DTYPES[t.dtype]


def _check_weight(w, x):
    if w is not None and (w.dtype != x.dtype or w.numel() != x.shape[-1] or not w.is_contiguous()):
        raise ValueError(f"norm weight must be a contiguous [{x.shape[-1]}] tensor of {x.dtype}")


def _row_layout(x: torch.Tensor):
    """(rows [R, n] with unit column stride, row pitch in elements) of the plain norm's input: a view of x when its
    rows are evenly spaced without overlap (a column slice of a wider projection is read in place; smel/norm.py
    reads such views the same way, :148-154), else a packed copy."""
    n = x.shape[-1]
    try:
        rows = x.view(-1, n)
    except RuntimeError:          # leading dims not flattenable into one stride
        rows = None
    if rows is None or rows.stride(1) != 1 or (rows.shape[0] > 1 and rows.stride(0) < n):
        rows = x.reshape(-1, n).contiguous()
    return rows, (rows.stride(0) if rows.shape[0] > 1 else n)


def _packed(t: torch.Tensor) -> torch.Tensor:
    """t as a packed [R, n] tensor (a view when t already is one)."""
    return t.reshape(-1, t.shape[-1]).contiguous()


class _NormFn(torch.autograd.Function):
    """forward(kind, eps, w_mode, w, a, b): kind "rms" (a = x), "add" (a = h, b = x; returns s and y) or "gated"
    (a = x, b = z). w_mode: 0 no weight, 1 w, 2 (1 + w)."""

    @staticmethod
    def forward(ctx, kind, eps, w_mode, w, a, b):
        _lib.require_device(a, b, w)
        _check_weight(w, a)
        dt, stream, p = _dtype_code(a), _lib.stream(), _lib.ptr
        ctx.kind, ctx.w_mode = kind, w_mode
        ctx.set_materialize_grads(False)
        if kind == _RMS:
            x2, pitch = _row_layout(a)
            R, n = x2.shape
            y = torch.empty(a.shape, device=a.device, dtype=a.dtype)
            rstd = torch.empty(R, device=a.device, dtype=torch.float32)
            _lib.call("smel_rmsnorm_fwd", p(x2), R, n, pitch, p(w), w_mode, float(eps), dt, p(y), p(rstd), stream)
            ctx.save_for_backward(x2, w, rstd)
            ctx.pitch, ctx.shapes = pitch, (a.shape,)
            return y
        a2, b2 = _packed(a), _packed(b)
        R, n = a2.shape
        rstd = torch.empty(R, device=a.device, dtype=torch.float32)
        y = torch.empty(a.shape, device=a.device, dtype=a.dtype)
        if kind == _ADD:
            s = torch.empty(a.shape, device=a.device, dtype=a.dtype)
            _lib.call("smel_add_rmsnorm_fwd", p(a2), p(b2), R, n, p(w), w_mode, float(eps), dt, p(s), p(y), p(rstd),
                      stream)
            ctx.save_for_backward(s, w, rstd)       # the norm's input is the rounded sum
            return s, y
        _lib.call("smel_gated_rmsnorm_fwd", p(a2), p(b2), R, n, p(w), float(eps), dt, p(y), p(rstd), stream)
        ctx.save_for_backward(a2, b2, w, rstd)
        ctx.shapes = (a.shape, b.shape)
        return y

    @staticmethod
    def backward(ctx, *grads):
        p, stream = _lib.ptr, _lib.stream()
        if ctx.kind == _RMS:
            x2, w, rstd = ctx.saved_tensors
            dy = grads[0]
            if dy is None:
                return None, None, None, None, None, None
            R, n = x2.shape
            dx = torch.empty(ctx.shapes[0], device=x2.device, dtype=x2.dtype)
            _lib.call("smel_rmsnorm_bwd", p(_packed(dy)), p(x2), R, n, ctx.pitch, p(w), ctx.w_mode, p(rstd), None,
                      _dtype_code(x2), p(dx), stream)
            return None, None, None, None, dx, None
        if ctx.kind == _ADD:
            # s feeds the norm and the residual stream: both inputs of the add get ds + the norm's dx (summed in
            # fp32 before one rounding); without a gradient through y it is ds alone
            s, w, rstd = ctx.saved_tensors
            ds, dy = grads
            if dy is None:
                return None, None, None, None, ds, ds
            s2 = s.reshape(-1, s.shape[-1])
            R, n = s2.shape
            d = torch.empty(s.shape, device=s.device, dtype=s.dtype)
            _lib.call("smel_rmsnorm_bwd", p(_packed(dy)), p(s2), R, n, n, p(w), ctx.w_mode, p(rstd),
                      p(_packed(ds)) if ds is not None else None, _dtype_code(s), p(d), stream)
            return None, None, None, None, d, d
        x2, z2, w, rstd = ctx.saved_tensors
        dout = grads[0]
        if dout is None:
            return None, None, None, None, None, None
        R, n = x2.shape
        dx = torch.empty(ctx.shapes[0], device=x2.device, dtype=x2.dtype)
        dz = torch.empty(ctx.shapes[1], device=z2.device, dtype=z2.dtype)
        _lib.call("smel_gated_rmsnorm_bwd", p(_packed(dout)), p(x2), p(z2), R, n, p(w), p(rstd), _dtype_code(x2),
                  p(dx), p(dz), stream)
        return None, None, None, None, dx, dz


def _w_mode(w, plus_one: bool) -> int:
    return 0 if w is None else (2 if plus_one else 1)


def supported(x, *weights):
    """Whether the kernels take this call: a GPU bf16/fp16 input of at most MAX_COLS columns whose norm weights are
    frozen, contiguous, of the input's dtype and shape [n_cols] (smel/norm.py:252-259)."""
    if not ENABLED or not x.is_cuda or x.dtype not in _DTYPES or x.shape[-1] > MAX_COLS:
        return False
    n = x.shape[-1]

    def fits(w):
        return w is None or (w.dtype == x.dtype and tuple(w.shape) == (n,) and w.is_contiguous()
                             and not w.requires_grad)
    return all(fits(w) for w in weights)


def rmsnorm(x, w, eps, plus_one):
    return _NormFn.apply(_RMS, eps, _w_mode(w, plus_one), w, x, None)


def add_rmsnorm(h, x, w, eps, plus_one):
    """(h + x, rmsnorm(h + x)): the residual add and the norm after it."""
    return _NormFn.apply(_ADD, eps, 2 if plus_one else 1, w, h, x)


def gated_rmsnorm(x, z, w, eps):
    return _NormFn.apply(_GATED, eps, 1, w, x, z)
