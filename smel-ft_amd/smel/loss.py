"""Chunked cross-entropy over a frozen lm_head (bf16 / fp32 rows, or int8 rows with per-row scales) that never holds
the [tokens, vocabulary] logits: the API of the reference's smel/loss.py (``LMHead``, ``chunked_ce``, ``_ce_chunk``,
``_ce_chunk_two_pass``; same arguments and results), on the HIP kernels of include/smel_loss.h.

Structure here:
  * an LMHead reads its rows through a row source (dense rows, or int8 rows dequantized per vocabulary chunk);
  * a token chunk is one sweep over the vocabulary chunks. Per vocabulary chunk: the logits GEMM h W_c^T (a library
    GEMM through torch), ``smel_ce_chunk_update`` (softcap, the online maximum and sum, the target's capped logit and
    cap derivative, the softmax terms in the rows' dtype; no host synchronisation), the gradient GEMM p W_c as a
    split K over column slices of the chunk, and ``smel_ce_acc_update`` (rescale and add in fp32);
  * the per-row state (maximum, sum, rescale, target logit and derivative, fp32 accumulator) is allocated once per
    call for the largest token chunk and reused by every chunk; the gradient rows go straight into one [N, H] output
    already divided by ``denom``.
The gradient is computed in the forward (lm_head is frozen) and handed back by the backward, as in the reference.
"""
from __future__ import annotations

import torch

from . import _lib as L
from .quant import dequant_int8_rows, quantize_int8_rows

_DT = {torch.bfloat16: 0, torch.float32: 1, torch.float16: 2}
SPLIT_PARTS = 8        # column slices of a vocabulary chunk in the gradient GEMM (its [tokens, H] output is small)


# --------------------------------------------------------------------------------------------------- the head


class _DenseRows:
    """Rows of a bf16 / fp32 head weight [V, H]."""

    def __init__(self, w: torch.Tensor):
        self.w = w

    def n(self) -> int:
        return self.w.shape[0]

    def span(self, v0: int, v1: int, dtype) -> torch.Tensor:
        return self.w[v0:v1].to(dtype)

    def take(self, idx: torch.Tensor, dtype) -> torch.Tensor:
        return self.w.index_select(0, idx).to(dtype)

    def moved(self, device):
        return _DenseRows(self.w.to(device))


class _Int8Rows:
    """Rows of an int8 head {"q": int8 [V, H], "scale": [V]} (smel/quant.py:97-105), dequantized where read."""

    def __init__(self, q: dict):
        self.q = q

    def n(self) -> int:
        return self.q["q"].shape[0]

    def span(self, v0: int, v1: int, dtype) -> torch.Tensor:
        return dequant_int8_rows(self.q["q"][v0:v1], self.q["scale"][v0:v1], dtype)

    def take(self, idx: torch.Tensor, dtype) -> torch.Tensor:
        return dequant_int8_rows(self.q["q"].index_select(0, idx), self.q["scale"].index_select(0, idx), dtype)

    def moved(self, device):
        return _Int8Rows({k: v.to(device) for k, v in self.q.items()})


class LMHead:
    """A frozen output head (smel/loss.py:12-47): ``weight`` (bf16 / fp32 rows [V, H]) or ``int8`` (the dict of
    quantize_int8_rows), read ``vocab_chunk`` rows at a time, with an optional final-logit softcap
    (z -> softcap tanh(z / softcap), Gemma)."""

    def __init__(self, weight: torch.Tensor | None = None, int8: dict | None = None, vocab_chunk: int = 32768,
                 softcap: float = 0.0):
        if (weight is None) == (int8 is None):
            raise AssertionError("LMHead takes exactly one of weight= or int8=")
        self.w, self.q = weight, int8
        self._src = _DenseRows(weight) if weight is not None else _Int8Rows(int8)
        self.vocab = self._src.n()
        self.vocab_chunk = vocab_chunk
        self.softcap = float(softcap or 0.0)

    @classmethod
    def from_weight(cls, w, int8=False, vocab_chunk=32768, softcap=0.0):
        kind = {"int8": quantize_int8_rows(w)} if int8 else {"weight": w}
        return cls(vocab_chunk=vocab_chunk, softcap=softcap, **kind)

    def to(self, device):
        src = self._src.moved(device)
        kind = {"weight": src.w} if isinstance(src, _DenseRows) else {"int8": src.q}
        return LMHead(vocab_chunk=self.vocab_chunk, softcap=self.softcap, **kind)

    def cap(self, z: torch.Tensor) -> torch.Tensor:
        c = self.softcap
        return torch.tanh(z / c) * c if c else z

    def rows(self, v0, v1, dtype):
        return self._src.span(v0, v1, dtype)

    def rows_at(self, idx, dtype):
        """The rows of the given vocabulary ids, as ``rows`` gives them."""
        return self._src.take(idx, dtype)

    def chunks(self):
        bounds = list(range(0, self.vocab, self.vocab_chunk)) + [self.vocab]
        return zip(bounds[:-1], bounds[1:])

    def logits(self, h):
        """Full logits [N, V] in fp32 (capped): a diagnostic, the loss never builds them."""
        out = torch.empty(h.shape[0], self.vocab, dtype=torch.float32, device=h.device)
        for v0, v1 in self.chunks():
            out[:, v0:v1] = self.cap(torch.mm(h, self.rows(v0, v1, h.dtype).t()).float())
        return out


# ------------------------------------------------------------------------------------------- one token chunk


def _split_parts(vc: int) -> int:
    """Column slices of a vocabulary chunk of vc columns for the split-K gradient GEMM: SPLIT_PARTS when every slice
    is at least 256 columns of whole 8-column groups, else 1."""
    return SPLIT_PARTS if vc % (8 * SPLIT_PARTS) == 0 and vc >= 256 * SPLIT_PARTS else 1


class _RowState:
    """Per-row state of one token chunk, allocated for up to ``cap`` rows and reused chunk after chunk."""

    def __init__(self, cap: int, H: int, need_grad: bool, device):
        f = lambda *s: torch.empty(*s, dtype=torch.float32, device=device)
        self.m, self.s, self.r, self.tl, self.td = f(cap), f(cap), f(cap), f(cap), f(cap)
        self.acc = f(cap, H) if need_grad else None

    def start(self, n: int, m0: torch.Tensor | None = None):
        """Views for n rows, reset for a sweep (m0: a preset running maximum, the two-pass form's second pass)."""
        v = [t[:n] for t in (self.m, self.s, self.r, self.tl, self.td)]
        m, s, r, tl, td = v
        if m0 is None:
            m.fill_(-float("inf"))
        else:
            m.copy_(m0)
        s.zero_()
        tl.zero_()
        td.fill_(1.0)
        acc = None
        if self.acc is not None:
            acc = self.acc[:n]
            acc.zero_()
        return m, s, r, tl, td, acc


def _sweep(h, head: LMHead, tgt, need_grad: bool, st: _RowState, m0=None):
    """One pass over the vocabulary for the rows h [n, H]: returns (m, s, tgt_logit, tgt_d, acc) after the last
    chunk (acc = sum_v softmax-term_v W_v, scaled to the final maximum; None without need_grad)."""
    n, H = h.shape
    dt = _DT[h.dtype]
    m, s, r, tl, td, acc = st.start(n, m0)
    stream = L.stream()
    for v0, v1 in head.chunks():
        W = head.rows(v0, v1, h.dtype).contiguous()
        vc = v1 - v0
        lg = torch.mm(h, W.t())                         # rounded to the rows' dtype, as the reference's h @ W.t()
        parts = _split_parts(vc) if need_grad else 1
        p = torch.empty(parts, n, vc // parts, dtype=h.dtype, device=h.device) if need_grad else None
        L.call("smel_ce_chunk_update", L.ptr(lg), n, vc, lg.stride(0), v0, L.ptr(tgt), head.softcap, dt,
               int(need_grad), L.ptr(m), L.ptr(s), L.ptr(tl), L.ptr(td), L.ptr(p), parts, L.ptr(r), stream)
        if need_grad:
            pw = torch.bmm(p, W.view(parts, vc // parts, H))   # slice k: p_k W_k, [parts, n, H]
            L.call("smel_ce_acc_update", L.ptr(acc), L.ptr(r), L.ptr(pw), parts, n, H, dt, stream)
    return m, s, tl, td, acc


def _finish(h, head: LMHead, tgt, m, s, tl, td, acc):
    """loss_sum = sum (lse - target logit); gradient rows = acc / s - tgt_d W[tgt] (a target outside [0, V) matches
    no row of the head: its logit and row count as zero, as in the reference's _ce_chunk)."""
    loss = (m + torch.log(s) - tl).sum()
    if acc is None:
        return loss, None
    ok = (tgt >= 0) & (tgt < head.vocab)
    rows = head.rows_at(torch.where(ok, tgt, torch.zeros_like(tgt)), h.dtype).float()
    return loss, acc / s[:, None] - (td * ok)[:, None] * rows


def _prep(h, tgt):
    L.require_device(h)
    if h.dtype not in _DT:
        raise ValueError(f"chunked CE takes bf16 / fp16 / fp32 rows, got {h.dtype}")
    return h.contiguous(), tgt.to(device=h.device, dtype=torch.int64).contiguous()


def _ce_chunk(h, head: LMHead, tgt, need_grad):
    """Loss sum and (optionally) d loss_sum / d h of one token chunk in ONE pass over the vocabulary
    (smel/loss.py:55-92): the gradient terms are accumulated under the same running maximum as the log-sum-exp and
    rescaled with it. The split-K gradient GEMM rounds each slice's product to the rows' dtype before the fp32 sum,
    where the reference rounds the one product."""
    h, tgt = _prep(h, tgt)
    st = _RowState(h.shape[0], h.shape[1], need_grad, h.device)
    return _finish(h, head, tgt, *_sweep(h, head, tgt, need_grad, st))


def _ce_chunk_two_pass(h, head: LMHead, tgt, need_grad):
    """The same quantities in two passes over the vocabulary (the comparator of smel/loss.py:95-127): the first pass
    finds each row's final maximum, the second runs with that maximum preset, so no partial sum or gradient term is
    ever rescaled."""
    h, tgt = _prep(h, tgt)
    st = _RowState(h.shape[0], h.shape[1], need_grad, h.device)
    m = _sweep(h, head, tgt, False, st)[0].clone()
    if not need_grad:
        return _finish(h, head, tgt, m, st.s[:h.shape[0]], st.tl[:h.shape[0]], st.td[:h.shape[0]], None)
    return _finish(h, head, tgt, *_sweep(h, head, tgt, True, st, m0=m))


# ------------------------------------------------------------------------------------------------ the loss


class _ChunkedCE(torch.autograd.Function):
    """sum_t CE / denom over token chunks (smel/loss.py:130-146); the gradient rows, already divided by denom, are
    written into one output during the forward and returned, times the incoming gradient, by the backward."""

    @staticmethod
    def forward(ctx, h, head, tgt, denom, token_chunk, need_grad):
        h, tgt = _prep(h, tgt)
        N, H = h.shape
        st = _RowState(min(N, token_chunk), H, need_grad, h.device)
        grad = torch.empty_like(h) if need_grad else None
        total = torch.zeros((), dtype=torch.float32, device=h.device)
        for t0 in range(0, N, token_chunk):
            t1 = min(N, t0 + token_chunk)
            loss, g = _finish(h[t0:t1], head, tgt[t0:t1], *_sweep(h[t0:t1], head, tgt[t0:t1], need_grad, st))
            total += loss
            if need_grad:
                grad[t0:t1] = g / denom
        ctx.grad = grad
        return total / denom

    @staticmethod
    def backward(ctx, go):
        g = ctx.grad
        ctx.grad = None
        return g * go.to(g.dtype), None, None, None, None, None


def chunked_ce(h, head: LMHead, tgt, denom: float, token_chunk: int = 1024, need_grad: bool = True):
    """sum_t CE(h_t W^T, tgt_t) / denom (smel/loss.py:149-156). h: [N, H] (final-normed, supervised rows only),
    tgt: [N] long."""
    if h.shape[0] == 0:
        return h.sum() * 0.0
    grad = need_grad and h.requires_grad
    with torch.set_grad_enabled(grad and torch.is_grad_enabled()):
        return _ChunkedCE.apply(h, head, tgt, float(denom), int(token_chunk), grad)
