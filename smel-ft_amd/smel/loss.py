"""Chunked cross-entropy over a frozen lm_head (bf16 / fp32 rows, or int8 rows with per-row scales) that never holds
the [tokens, vocabulary] logits: the API of the reference's smel/loss.py (``LMHead``, ``chunked_ce``, ``_ce_chunk``,
``_ce_chunk_two_pass``; same arguments and results), on the HIP kernels of include/smel_loss.h.

Structure here:
  * a pass covers a block of token rows; per vocabulary chunk, ``smel_ce_logits`` runs the logits GEMM on MFMA and,
    in its epilogue, the online softmax bookkeeping per 128-column window (maximum rounded up to a power of two, sum
    of exponentials, the softmax terms written in the rows' dtype, the target's logit), ``smel_ce_stats`` folds the
    windows into each row's running maximum and sum (every rescale an exact power of two) and ``smel_ce_grad`` runs
    the gradient GEMM p W on MFMA, shifting each fragment of p to the running maximum as it is loaded and adding into
    the fp32 accumulator rescaled by the same power of two (the chunk's columns in two halves, the second half's sum
    kept apart and folded in by the next chunk); ``smel_ce_finish`` writes the loss rows and the gradient rows
    (acc / s - d W[target], scaled), ``smel_ce_loss_sum`` their sum;
  * the gradient GEMM reads the head transposed ([H][V]): a dense head whose dtype is the rows' is transposed once
    and kept with the head (it is frozen); other heads (int8, or another dtype) are converted per vocabulary chunk,
    as the reference's ``rows()`` does, and that chunk is transposed;
  * vocabulary chunks are ``vocab_chunk`` rounded up to 256 columns (the logits tile), and a pass takes at most
    ``token_chunk`` rows, so token_chunk x vocab_chunk bounds its buffers as in the reference (the softmax terms of a
    pass take rows x chunk values of the rows' dtype); a caller that leaves token_chunk at its default gets passes of
    up to 4096 rows (256 MB of bf16 terms at vocab_chunk 32768), where the GEMMs' row tiles fill the GPU. The rows are
    independent, so the results are those of the reference's chunking either way.
The gradient is computed in the forward (lm_head is frozen) and handed back by the backward, as in the reference.
"""
from __future__ import annotations

import torch

from . import _lib as L
from .quant import dequant_int8_rows, quantize_int8_rows

_DT = {torch.bfloat16: 0, torch.float32: 1, torch.float16: 2}
TILE_V = 256           # vocabulary columns of a logits tile; chunks are whole tiles
WIN = 128              # columns of one statistics window
ROWS_PER_PASS = 4096   # token rows of a pass when token_chunk is left at its default (the GEMMs fill the GPU there)


class _DefaultTokenChunk(int):
    """The default token_chunk of chunked_ce (1024, the reference's): a caller who left it has not bounded the rows
    of a pass, which may then take ROWS_PER_PASS rows."""


TOKEN_CHUNK_DEFAULT = _DefaultTokenChunk(1024)


def _rows_per_pass(N: int, token_chunk) -> int:
    """Token rows of one pass: at most ``token_chunk`` (it bounds a pass's buffers, the softmax terms
    [rows][vocab_chunk] and about 12 H bytes per row), or up to ROWS_PER_PASS when the caller left the default."""
    tc = int(token_chunk)
    if tc <= 0:
        raise ValueError(f"chunked_ce: token_chunk must be positive, got {tc}")
    if isinstance(token_chunk, _DefaultTokenChunk):
        tc = max(tc, ROWS_PER_PASS)
    return min(N, tc)


def _round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


# --------------------------------------------------------------------------------------------------- the head


class _DenseRows:
    """Rows of a bf16 / fp16 / fp32 head weight [V, H]."""

    def __init__(self, w: torch.Tensor):
        self.w = w

    def n(self) -> int:
        return self.w.shape[0]

    def span(self, v0: int, v1: int, dtype) -> torch.Tensor:
        return self.w[v0:v1].to(dtype)

    def take(self, idx: torch.Tensor, dtype) -> torch.Tensor:
        return self.w.index_select(0, idx).to(dtype)

    def native(self, dtype):
        """The weight itself when the kernels can read it as rows of `dtype` in place, else None."""
        w = self.w
        if w.dtype != dtype or not w.is_cuda or w.stride(1) != 1:
            return None
        e = w.element_size()
        if (w.shape[1] * e) % 16 or (w.stride(0) * e) % 16 or w.data_ptr() % 16:
            return None
        return w

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

    def native(self, dtype):
        return None

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
        self._wt = {}    # dtype -> (key, transposed head [H][Vp]) for a dense head read in place

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

    # ---- what the kernels read
    def _kernel_chunks(self):
        """Vocabulary chunks of the kernels: vocab_chunk rounded up to whole logits tiles."""
        step = _round_up(max(1, min(self.vocab_chunk, self.vocab)), TILE_V)
        return [(v0, min(self.vocab, v0 + step)) for v0 in range(0, self.vocab, step)], step

    def _transposed(self, w: torch.Tensor) -> torch.Tensor:
        """The head [V, H] transposed to [H, Vp] (Vp = V rounded up to 8, zero columns past V), made once."""
        key = (w.data_ptr(), w._version, tuple(w.shape), w.dtype)
        got = self._wt.get(w.dtype)
        if got is not None and got[0] == key:
            return got[1]
        V, H = w.shape
        wt = torch.empty(H, _round_up(V, 8), dtype=w.dtype, device=w.device)
        L.call("smel_ce_transpose", L.ptr(w), V, H, w.stride(0), L.ptr(wt), wt.stride(0), _DT[w.dtype], L.stream())
        self._wt[w.dtype] = (key, wt)
        return wt


# ------------------------------------------------------------------------------------------------ one pass


class _Pass:
    """Scratch of one pass over n token rows: per-row state, window statistics, softmax terms, accumulator."""

    def __init__(self, n: int, H: int, vcp: int, dtype, need_grad: bool, device):
        f = lambda *s: torch.empty(*s, dtype=torch.float32, device=device)
        nwin = vcp // WIN
        self.n = n
        self.m, self.s, self.tz, self.td, self.r, self.loss = (f(n) for _ in range(6))
        self.win_e, self.win_s = f(nwin, n), f(nwin, n)
        self.shift = torch.empty(nwin, n, dtype=torch.uint8, device=device)
        self.P = torch.empty(n, vcp, dtype=dtype, device=device) if need_grad else None
        self.acc = f(n, H) if need_grad else None
        self.part = f(2, n, H) if need_grad else None     # the second K halves' partials, by chunk parity
        self.last = 0                                       # chunks of the last sweep


def _sweep(h, head: LMHead, tgt, need_grad: bool, ps: _Pass, m0=None):
    """One pass over the vocabulary for the rows h [n, H]: the per-row state and (need_grad) the accumulator."""
    n, H = h.shape
    dt, st, p = _DT[h.dtype], L.stream(), L.ptr
    L.call("smel_ce_begin", p(ps.m), p(ps.s), p(ps.tz), p(ps.td), p(m0), n, st)
    native = head._src.native(h.dtype)
    chunks, _ = head._kernel_chunks()
    for i, (v0, v1) in enumerate(chunks):
        vc = v1 - v0
        if native is not None:
            W, ldw = native[v0:v1], native.stride(0)
        else:
            W = head.rows(v0, v1, h.dtype).contiguous()
            ldw = W.stride(0)
        nwin = _round_up(vc, TILE_V) // WIN
        P = ps.P if need_grad else None
        L.call("smel_ce_logits", p(W), ldw, vc, v0, p(h), h.stride(0), n, H, p(tgt), head.softcap, dt, p(P),
               P.stride(0) if need_grad else 0, p(ps.win_e), p(ps.win_s), n, p(ps.tz), p(ps.td), st)
        L.call("smel_ce_stats", p(ps.win_e), p(ps.win_s), nwin, n, n, p(ps.m), p(ps.s), p(ps.shift), p(ps.r), st)
        if need_grad:
            if native is not None:
                wt = head._transposed(native)
                WT, ldwt = wt[:, v0:], wt.stride(0)
            else:
                WT = torch.empty(H, _round_up(vc, 8), dtype=h.dtype, device=h.device)
                L.call("smel_ce_transpose", p(W), vc, H, ldw, p(WT), WT.stride(0), dt, st)
                ldwt = WT.stride(0)
            L.call("smel_ce_grad", p(WT), ldwt, H, p(ps.P), ps.P.stride(0), vc, p(ps.shift), n, p(ps.r), n, dt,
                   i, p(ps.acc), p(ps.part), st)
    ps.last = len(chunks) - 1


def _finish(h, head: LMHead, tgt, ps: _Pass, need_grad: bool, gscale: float = 1.0, g=None):
    """Loss rows into ps.loss and (need_grad) gradient rows gscale (acc / s - d W[target]) into g (default: a new
    fp32 [n, H]); a target outside [0, V) matches no row of the head (its logit and row count as zero, as in the
    reference's _ce_chunk)."""
    n, H = h.shape
    dt, p = _DT[h.dtype], L.ptr
    W, ldw, trows = None, 0, None
    if need_grad:
        native = head._src.native(h.dtype)
        if native is not None:
            W, ldw = native, native.stride(0)
        else:
            ok = (tgt >= 0) & (tgt < head.vocab)
            trows = head.rows_at(torch.where(ok, tgt, torch.zeros_like(tgt)), h.dtype).contiguous()
        if g is None:
            g = torch.empty(n, H, dtype=torch.float32, device=h.device)
    part = ps.part[ps.last % 2] if need_grad else None
    L.call("smel_ce_finish", p(ps.m), p(ps.s), p(ps.tz), p(ps.td), p(ps.acc), p(part), p(W), ldw, p(trows), p(tgt),
           head.vocab, n, H, dt, float(gscale), p(g), g.stride(0) if g is not None else 0,
           _DT[g.dtype] if g is not None else 0, p(ps.loss), L.stream())
    return g


def _prep(h, tgt):
    L.require_device(h)
    if h.dtype not in _DT:
        raise ValueError(f"chunked CE takes bf16 / fp16 / fp32 rows, got {h.dtype}")
    h = h.contiguous()
    if (h.shape[1] * h.element_size()) % 16:
        raise ValueError(f"chunked CE takes rows of whole 16-byte runs (hidden size {h.shape[1]} in {h.dtype})")
    return h, tgt.to(device=h.device, dtype=torch.int64).contiguous()


def _loss_sum(ps: _Pass, total: torch.Tensor, scale: float, accumulate: bool):
    L.call("smel_ce_loss_sum", L.ptr(ps.loss), ps.n, float(scale), int(accumulate), L.ptr(total), L.stream())


def _one_chunk(h, head: LMHead, tgt, need_grad, two_pass: bool):
    h, tgt = _prep(h, tgt)
    n, H = h.shape
    _, vcp = head._kernel_chunks()
    total = torch.empty((), dtype=torch.float32, device=h.device)
    ps = _Pass(n, H, vcp, h.dtype, need_grad, h.device)
    m0 = None
    if two_pass:
        _sweep(h, head, tgt, False, ps)
        m0 = ps.m.clone()
    _sweep(h, head, tgt, need_grad, ps, m0=m0)
    g = _finish(h, head, tgt, ps, need_grad)
    _loss_sum(ps, total, 1.0, False)
    return total, g


def _ce_chunk(h, head: LMHead, tgt, need_grad):
    """Loss sum and (optionally) d loss_sum / d h (fp32) of one token chunk in ONE pass over the vocabulary
    (smel/loss.py:55-92): the gradient terms are accumulated under the same running maximum as the log-sum-exp and
    rescaled with it."""
    return _one_chunk(h, head, tgt, need_grad, False)


def _ce_chunk_two_pass(h, head: LMHead, tgt, need_grad):
    """The same quantities in two passes over the vocabulary (the comparator of smel/loss.py:95-127): the first pass
    finds each row's final maximum, the second runs with that maximum preset, so no partial sum or gradient term is
    ever rescaled."""
    return _one_chunk(h, head, tgt, need_grad, True)


# ------------------------------------------------------------------------------------------------ the loss


class _ChunkedCE(torch.autograd.Function):
    """sum_t CE / denom over token passes (smel/loss.py:130-146); the gradient rows, already divided by denom, are
    written into one output during the forward and returned, times the incoming gradient, by the backward."""

    @staticmethod
    def forward(ctx, h, head, tgt, denom, rows, need_grad):
        h, tgt = _prep(h, tgt)
        N, H = h.shape
        _, vcp = head._kernel_chunks()
        grad = torch.empty_like(h) if need_grad else None
        total = torch.empty((), dtype=torch.float32, device=h.device)
        ps = _Pass(rows, H, vcp, h.dtype, need_grad, h.device)
        for t0 in range(0, N, rows):
            t1 = min(N, t0 + rows)
            if t1 - t0 != ps.n:
                ps = _Pass(t1 - t0, H, vcp, h.dtype, need_grad, h.device)
            _sweep(h[t0:t1], head, tgt[t0:t1], need_grad, ps)
            _finish(h[t0:t1], head, tgt[t0:t1], ps, need_grad, 1.0 / denom, grad[t0:t1] if need_grad else None)
            _loss_sum(ps, total, 1.0 / denom, t0 > 0)
        ctx.grad = grad
        return total

    @staticmethod
    def backward(ctx, go):
        g = ctx.grad
        ctx.grad = None
        go = go.to(device=g.device, dtype=torch.float32).contiguous()
        L.call("smel_ce_scale", L.ptr(g), g.numel(), _DT[g.dtype], L.ptr(go), L.stream())
        return g, None, None, None, None, None


def chunked_ce(h, head: LMHead, tgt, denom: float, token_chunk: int = TOKEN_CHUNK_DEFAULT, need_grad: bool = True):
    """sum_t CE(h_t W^T, tgt_t) / denom (smel/loss.py:149-156). h: [N, H] (final-normed, supervised rows only),
    tgt: [N] long. A pass over the vocabulary takes at most ``token_chunk`` rows when the caller sets it."""
    if h.shape[0] == 0:
        return h.sum() * 0.0
    rows = _rows_per_pass(h.shape[0], token_chunk)
    grad = need_grad and h.requires_grad
    with torch.set_grad_enabled(grad and torch.is_grad_enabled()):
        return _ChunkedCE.apply(h, head, tgt, float(denom), rows, grad)
