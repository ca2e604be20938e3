"""int4 group-wise format of the frozen experts (API of smel/quant.py), dequant through the HIP kernel.

Format (the reference's, smel/quant.py:14-44): q uint8 [..., K/2] with the even column in the low nibble, scale and
zero bf16 [..., K/group], w = q*scale + zero. ``dequant_int4`` is the MI355X kernel (fp32 math, one
round-to-nearest-even, as the reference's GPU kernel smel/quant.py:51-67). ``quantize_int4`` is the offline packer of
the reference's pack stage (not on the hot path): it always runs the HIP kernel ``smel_quantize_int4`` (one thread
per group, the reference's fp32 steps in its order); a host tensor is copied to the current GPU for it and the
result copied back, so there is no CPU quantizer in this package.
"""
from __future__ import annotations

import torch

from . import _lib as L


_QDT = {torch.bfloat16: 0, torch.float32: 1, torch.float16: 2}


def quantize_int4(w: torch.Tensor, group: int = 64, clip_search=(1.0, 0.95, 0.9, 0.85, 0.8)) -> dict:
    """w [..., K] -> {"q": uint8 [..., K/2], "scale": bf16 [..., K/group], "zero": bf16 [..., K/group]}
    (smel/quant.py:14-44): per group, the [min, max] range shrunk about its midpoint by the clip factor with the
    smallest squared error (a later factor must be strictly better). One HIP launch for the whole tensor; a host
    tensor goes through the current GPU and the result comes back on the host."""
    K = w.shape[-1]
    assert K % group == 0 and group % 2 == 0, f"K={K} must be a multiple of the (even) group {group}"
    if not w.is_cuda:
        if not torch.cuda.is_available():
            raise RuntimeError("quantize_int4 runs on the GPU (HIP kernel smel_quantize_int4); no GPU is visible")
        return {k: v.cpu() for k, v in quantize_int4(w.cuda(), group, clip_search).items()}
    clip = list(clip_search or (1.0,))
    if w.dtype not in _QDT:
        w = w.float()
    wc = w.contiguous()
    rows = wc.numel() // K
    q = torch.empty(*w.shape[:-1], K // 2, dtype=torch.uint8, device=w.device)
    scale = torch.empty(*w.shape[:-1], K // group, dtype=torch.bfloat16, device=w.device)
    zero = torch.empty_like(scale)
    if rows:
        cf = (L.f32 * len(clip))(*clip)
        L.call("smel_quantize_int4", L.ptr(wc), _QDT[wc.dtype], rows, K, group, cf, len(clip), L.ptr(q),
               L.ptr(scale), L.ptr(zero), L.stream())
    return {"q": q, "scale": scale, "zero": zero}


def dequant_int4(q: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor, dtype=torch.bfloat16) -> torch.Tensor:
    """int4 -> ``dtype`` (bf16 or fp32) on the GPU (smel/quant.py:74-84)."""
    if dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"dequant_int4: unsupported output dtype {dtype}")
    L.require_device(q, scale, zero)
    q, scale, zero = q.contiguous(), scale.contiguous(), zero.contiguous()
    K = q.shape[-1] * 2
    G = scale.shape[-1]
    out = torch.empty(*q.shape[:-1], K, device=q.device, dtype=dtype)
    rows = q.numel() // max(1, q.shape[-1])
    L.call("smel_dequant_int4", L.ptr(q), L.ptr(scale), L.ptr(zero), L.ptr(out), rows, K, K // G,
           int(dtype == torch.float32), L.stream())
    return out


def dequant_int4_torch(q, scale, zero, dtype=torch.bfloat16):
    """The reference's torch fallback semantics (smel/quant.py:87-94: product and add rounded in ``dtype``), kept
    for API compatibility; not used by the kernels."""
    K = q.shape[-1] * 2
    G = scale.shape[-1]
    w = torch.stack((q & 0xF, q >> 4), dim=-1).reshape(*q.shape[:-1], G, K // G).to(dtype)
    w = w * scale.unsqueeze(-1).to(dtype) + zero.unsqueeze(-1).to(dtype)
    return w.reshape(*q.shape[:-1], K)


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.float(), b.float()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def quantize_int8_rows(w: torch.Tensor):
    """Symmetric per-row int8 of a dense matrix (lm_head), smel/quant.py:97-101: scale = max(|w|) / 127 (at least
    1e-12), q = clamp(round(w / scale), -127, 127); scale stored as bf16."""
    s = (w.float().abs().amax(-1, keepdim=True) / 127).clamp_min(1e-12)
    q = torch.round(w.float() / s).clamp_(-127, 127).to(torch.int8)
    return {"q": q, "scale": s.squeeze(-1).to(torch.bfloat16)}


def dequant_int8_rows(q, scale, dtype=torch.bfloat16):
    """q * scale in `dtype` (smel/quant.py:104-105)."""
    return q.to(dtype) * scale.unsqueeze(-1).to(dtype)
