"""Chunked cross-entropy over a frozen lm_head (bf16 or int8 rows) without materializing [T, vocab] logits
(the reference's smel/loss.py: ``LMHead``, ``chunked_ce``, ``_ce_chunk``, ``_ce_chunk_two_pass``, same arguments
and results).

One pass over the vocabulary per token chunk gives the loss and the gradient w.r.t. the hidden states (lm_head is
frozen): per vocabulary chunk, the logits GEMM h W_c^T and the gradient GEMM p W_c are library GEMMs (rocBLAS /
hipBLASLt through torch), and everything between them — the final-logit softcap, the running max and sum of the
online log-sum-exp, the softmax terms (times the cap derivative) in the rows' dtype, the target's logit and cap
derivative, the accumulator's rescale — runs in the HIP kernels of include/smel_loss.h, without the reference's
host synchronisations (``inside.any()`` / ``nonzero`` per chunk). Peak memory: one [token_chunk, vocab_chunk]
logits tile and its softmax terms.
"""
from __future__ import annotations

import torch

from . import _lib as L
from .quant import dequant_int8_rows, quantize_int8_rows

_DT = {torch.bfloat16: 0, torch.float32: 1, torch.float16: 2}


class LMHead:
    """smel/loss.py:12-52: a frozen head as bf16 (or fp32) rows or int8 rows with per-row scales."""

    def __init__(self, weight: torch.Tensor | None = None, int8: dict | None = None, vocab_chunk: int = 32768,
                 softcap: float = 0.0):
        assert (weight is None) != (int8 is None)
        self.w, self.q = weight, int8
        self.vocab = weight.shape[0] if weight is not None else int8["q"].shape[0]
        self.vocab_chunk = vocab_chunk
        self.softcap = float(softcap or 0.0)

    @classmethod
    def from_weight(cls, w, int8=False, vocab_chunk=32768, softcap=0.0):
        if int8:
            return cls(int8=quantize_int8_rows(w), vocab_chunk=vocab_chunk, softcap=softcap)
        return cls(weight=w, vocab_chunk=vocab_chunk, softcap=softcap)

    def to(self, device):
        if self.w is not None:
            return LMHead(weight=self.w.to(device), vocab_chunk=self.vocab_chunk, softcap=self.softcap)
        return LMHead(int8={k: v.to(device) for k, v in self.q.items()}, vocab_chunk=self.vocab_chunk,
                      softcap=self.softcap)

    def cap(self, z: torch.Tensor) -> torch.Tensor:
        return self.softcap * torch.tanh(z / self.softcap) if self.softcap else z

    def rows(self, v0, v1, dtype):
        if self.w is not None:
            return self.w[v0:v1].to(dtype)
        return dequant_int8_rows(self.q["q"][v0:v1], self.q["scale"][v0:v1], dtype)

    def rows_at(self, idx, dtype):
        """The rows of the given vocabulary ids, as ``rows`` would give them."""
        if self.w is not None:
            return self.w[idx].to(dtype)
        return dequant_int8_rows(self.q["q"][idx], self.q["scale"][idx], dtype)

    def chunks(self):
        for v0 in range(0, self.vocab, self.vocab_chunk):
            yield v0, min(self.vocab, v0 + self.vocab_chunk)

    def logits(self, h):
        return torch.cat([self.cap(torch.mm(h, self.rows(v0, v1, h.dtype).t()).float()) for v0, v1 in self.chunks()],
                         dim=-1)


SPLIT_PARTS = 8        # slices of the vocabulary chunk in the gradient GEMM (its output alone has too few tiles)


def _split_parts(vc: int) -> int:
    """Slices of a vocabulary chunk of vc columns for the split-K gradient GEMM: SPLIT_PARTS when each slice is
    still at least 256 columns of whole 8-column groups, else 1."""
    k = SPLIT_PARTS
    return k if vc % (8 * k) == 0 and vc // k >= 256 else 1


def _ce_chunk(h, head: LMHead, tgt, need_grad):
    """Loss sum and (optionally) d loss_sum / d h for one token chunk in ONE pass over the vocabulary
    (smel/loss.py:55-92): the gradient sum_v softmax_v dcap_v W_v is accumulated with the same running maximum as the
    log-sum-exp, the target row subtracted at the end. The gradient GEMM of each vocabulary chunk runs as a split K
    (its [tokens, H] output alone gives too few tiles): its slices' products are rounded to the rows' dtype each and
    summed in fp32, where the reference rounds the one product."""
    L.require_device(h)
    if h.dtype not in _DT:
        raise ValueError(f"chunked CE takes bf16 / fp16 / fp32 rows, got {h.dtype}")
    n, H = h.shape
    dt = _DT[h.dtype]
    dev = h.device
    tgt = tgt.to(torch.int64).contiguous()
    m = torch.full((n,), -float("inf"), device=dev)
    s = torch.zeros(n, device=dev)
    r = torch.empty(n, device=dev)
    tgt_logit = torch.zeros(n, device=dev)
    tgt_d = torch.ones(n, device=dev)
    acc = torch.zeros(n, H, device=dev) if need_grad else None
    st = L.stream()
    for v0, v1 in head.chunks():
        W = head.rows(v0, v1, h.dtype).contiguous()
        lg = torch.mm(h, W.t())                      # [n, vc] in the rows' dtype, as the reference's h @ W.t()
        vc = v1 - v0
        parts = _split_parts(vc) if need_grad else 1
        p = torch.empty(parts, n, vc // parts, device=dev, dtype=h.dtype) if need_grad else None
        L.call("smel_ce_chunk_update", L.ptr(lg), n, vc, lg.stride(0), v0, L.ptr(tgt), head.softcap, dt,
               int(need_grad), L.ptr(m), L.ptr(s), L.ptr(tgt_logit), L.ptr(tgt_d), L.ptr(p), parts, L.ptr(r), st)
        if need_grad:
            # split K: [parts, n, vc/parts] x [parts, vc/parts, H] (both contiguous) -> [parts, n, H]
            pw = torch.bmm(p, W.view(parts, vc // parts, H))
            L.call("smel_ce_acc_update", L.ptr(acc), L.ptr(r), L.ptr(pw), parts, n, H, dt, st)
    lse = m + s.log()
    loss = (lse - tgt_logit).sum()
    if not need_grad:
        return loss, None
    gh = acc / s[:, None] - tgt_d[:, None] * head.rows_at(tgt, h.dtype).float()
    return loss, gh


def _ce_chunk_two_pass(h, head: LMHead, tgt, need_grad):
    """Loss sum and (optionally) d loss_sum / d h for one token chunk in two passes over the vocabulary, as torch
    ops (the reference's comparator, smel/loss.py:95-127): the log-sum-exp first, then the exact softmax per chunk.
    It shares no code with ``_ce_chunk``."""
    n = h.shape[0]
    dev = h.device
    tgt = tgt.to(torch.int64)
    rows = torch.arange(n, device=dev)
    m = torch.full((n,), -float("inf"), device=dev)
    s = torch.zeros(n, device=dev)
    tgt_logit = torch.zeros(n, device=dev)
    for v0, v1 in head.chunks():
        lg = head.cap(torch.mm(h, head.rows(v0, v1, h.dtype).t()).float())
        nm = torch.maximum(m, lg.amax(-1))
        s = s * (m - nm).exp() + (lg - nm[:, None]).exp().sum(-1)
        m = nm
        inside = (tgt >= v0) & (tgt < v1)
        tgt_logit = torch.where(inside, lg[rows, (tgt - v0).clamp(0, v1 - v0 - 1)], tgt_logit)
    lse = m + s.log()
    loss = (lse - tgt_logit).sum()
    if not need_grad:
        return loss, None
    gh = torch.zeros(h.shape, device=dev, dtype=torch.float32)
    for v0, v1 in head.chunks():
        W = head.rows(v0, v1, h.dtype)
        lg = head.cap(torch.mm(h, W.t()).float())
        p = (lg - lse[:, None]).exp()
        inside = (tgt >= v0) & (tgt < v1)
        p[rows, (tgt - v0).clamp(0, v1 - v0 - 1)] -= inside.float()
        if head.softcap:
            p = p * (1 - (lg / head.softcap) ** 2)
        gh += torch.mm(p.to(h.dtype), W)
    return loss, gh


class _ChunkedCE(torch.autograd.Function):
    """smel/loss.py:130-146: the gradient is computed in the forward and handed back by backward."""

    @staticmethod
    def forward(ctx, h, head, tgt, denom, token_chunk, need_grad):
        total = torch.zeros((), device=h.device)
        grads = [] if need_grad else None
        for t0 in range(0, h.shape[0], token_chunk):
            l, g = _ce_chunk(h[t0:t0 + token_chunk], head, tgt[t0:t0 + token_chunk], need_grad)
            total += l
            if need_grad:
                grads.append(g)
        if need_grad:
            ctx.grad = (torch.cat(grads) / denom).to(h.dtype) if grads else torch.zeros_like(h)
        return total / denom

    @staticmethod
    def backward(ctx, go):
        return ctx.grad * go.to(ctx.grad.dtype), None, None, None, None, None


def chunked_ce(h, head: LMHead, tgt, denom: float, token_chunk: int = 1024, need_grad: bool = True):
    """sum_t CE(h_t W^T, tgt_t) / denom (smel/loss.py:149-156). h: [N, H] (final-normed, only supervised rows),
    tgt: [N] long."""
    if h.shape[0] == 0:
        return h.sum() * 0.0
    if need_grad and h.requires_grad:
        return _ChunkedCE.apply(h.contiguous(), head, tgt, float(denom), token_chunk, True)
    with torch.no_grad():
        return _ChunkedCE.apply(h.contiguous(), head, tgt, float(denom), token_chunk, False)
