"""Single-pass chunked CE (smel.loss over include/smel_loss.h) on the GPU: the reference's own three tests
(tests/test_loss_single_pass.py:23-63: against full fp32 logits with and without softcapping at 1e-4, bf16 single
pass against the two-pass comparator, the int8 head against its dequantized weight) and the fp64 oracle
(oracle/loss_ref.py) at a larger bf16 shape; a vocabulary that is not a multiple of the chunk, several token chunks,
a target in every chunk position (first, last column)."""
import pytest
import torch

from oracle import loss_ref as LR

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lm():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from smel import loss, quant
    return loss, quant


def full_ref(h, W, tgt, softcap, denom):
    h = h.detach().clone().requires_grad_(True)
    lg = h @ W.float().t()
    if softcap:
        lg = softcap * torch.tanh(lg / softcap)
    loss = torch.nn.functional.cross_entropy(lg, tgt, reduction="sum") / denom
    loss.backward()
    return loss.detach(), h.grad


@pytest.mark.parametrize("softcap", [0.0, 30.0])
def test_fp32_matches_full_logits(lm, softcap):
    loss_mod, _ = lm
    torch.manual_seed(0)
    n, H, V = 37, 64, 1000                      # V is not a multiple of the vocab chunk
    h = torch.randn(n, H, device="cuda") * 0.5
    W = torch.randn(V, H, device="cuda") * 0.2
    tgt = torch.randint(0, V, (n,), device="cuda")
    tgt[0], tgt[1], tgt[2] = 0, V - 1, 127      # first column, last column, last column of a chunk
    head = loss_mod.LMHead(weight=W, vocab_chunk=128, softcap=softcap)
    loss_ref, grad_ref = full_ref(h, W, tgt, softcap, denom=n)
    h_ = h.clone().requires_grad_(True)
    loss = loss_mod.chunked_ce(h_, head, tgt, denom=n, token_chunk=16)
    loss.backward()
    assert abs(loss.item() - loss_ref.item()) < 1e-4 * max(1.0, abs(loss_ref.item()))
    assert (h_.grad - grad_ref).norm() / grad_ref.norm() < 1e-4
    l64, g64 = LR.full_ce(h, W, tgt, softcap, denom=n)
    assert abs(loss.item() - float(l64)) < 1e-4 * max(1.0, abs(float(l64)))
    assert (h_.grad.double().cpu() - g64).norm() / g64.norm() < 1e-4


def test_bf16_matches_two_pass(lm):
    loss_mod, _ = lm
    torch.manual_seed(1)
    n, H, V = 300, 128, 5000
    h = (torch.randn(n, H, device="cuda") * 0.5).bfloat16()
    W = (torch.randn(V, H, device="cuda") * 0.2).bfloat16()
    tgt = torch.randint(0, V, (n,), device="cuda")
    for softcap in (0.0, 30.0):
        head = loss_mod.LMHead(weight=W, vocab_chunk=1024, softcap=softcap)
        l1, g1 = loss_mod._ce_chunk(h, head, tgt, True)
        l2, g2 = loss_mod._ce_chunk_two_pass(h, head, tgt, True)
        assert abs(l1.item() - l2.item()) / abs(l2.item()) < 1e-3
        assert (g1 - g2).norm() / g2.norm() < 2e-2
        l64, g64 = LR.full_ce(h, W, tgt, softcap)
        assert abs(l1.item() - float(l64)) / abs(float(l64)) < 1e-3
        assert (g1.double().cpu() - g64).norm() / g64.norm() < 3e-2    # bf16 logits and probabilities


def test_int8_head_runs_and_matches_its_dequantized_weight(lm):
    loss_mod, quant = lm
    torch.manual_seed(2)
    n, H, V = 64, 96, 700
    h = torch.randn(n, H, device="cuda") * 0.5
    W = torch.randn(V, H, device="cuda") * 0.2
    tgt = torch.randint(0, V, (n,), device="cuda")
    q = {k: v.cuda() for k, v in quant.quantize_int8_rows(W).items()}
    w_dq = quant.dequant_int8_rows(q["q"], q["scale"], torch.float32)
    loss_q = loss_mod.chunked_ce(h, loss_mod.LMHead(int8=q, vocab_chunk=256), tgt, denom=n, token_chunk=32,
                                 need_grad=False)
    loss_dq = loss_mod.chunked_ce(h, loss_mod.LMHead(weight=w_dq), tgt, denom=n, token_chunk=32, need_grad=False)
    assert abs(loss_q.item() - loss_dq.item()) < 1e-3 * abs(loss_dq.item())


def test_repeatable_and_empty(lm):
    loss_mod, _ = lm
    torch.manual_seed(3)
    h = (torch.randn(130, 64, device="cuda")).bfloat16().requires_grad_(True)
    W = (torch.randn(777, 64, device="cuda") * 0.2).bfloat16()
    tgt = torch.randint(0, 777, (130,), device="cuda")
    head = loss_mod.LMHead(weight=W, vocab_chunk=100)
    a = loss_mod.chunked_ce(h, head, tgt, denom=130.0, token_chunk=64)
    a.backward()
    ga = h.grad.clone()
    h.grad = None
    b = loss_mod.chunked_ce(h, head, tgt, denom=130.0, token_chunk=64)
    b.backward()
    assert torch.equal(a, b) and torch.equal(ga, h.grad)
    e = loss_mod.chunked_ce(h[:0], head, tgt[:0], denom=1.0)
    assert e.item() == 0.0
