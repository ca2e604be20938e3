"""CPU restatement of the chunked cross-entropy's result (smel/loss.py:149-156) — TEST INFRASTRUCTURE ONLY.

What the reference's single-pass chunked CE computes is the plain cross-entropy of the full logits: loss =
sum_t (logsumexp(cap(h_t W^T)) - cap(h_t W^T)[tgt_t]) / denom, with cap(z) = c tanh(z / c) when softcapping, and its
gradient w.r.t. h. This module computes it from the full logits in fp64 (torch on the CPU, autograd for the
gradient), the comparator the reference's own tests use (tests/test_loss_single_pass.py:12-20).

PINNED (tests/test_loss_oracle.py): torch.nn.functional.cross_entropy against a per-row numpy log-sum-exp;
the softcapped gradient against central finite differences.
"""
from __future__ import annotations

import torch


def full_ce(h, W, tgt, softcap=0.0, denom=1.0):
    """(loss, dloss/dh) in fp64 from the full logits."""
    h64 = h.detach().double().cpu().requires_grad_(True)
    lg = h64 @ W.detach().double().cpu().t()
    if softcap:
        lg = softcap * torch.tanh(lg / softcap)
    loss = torch.nn.functional.cross_entropy(lg, tgt.cpu().long(), reduction="sum") / denom
    loss.backward()
    return loss.detach(), h64.grad
