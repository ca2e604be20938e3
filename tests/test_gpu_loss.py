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


def rounded_full_ce(h, W, tgt, softcap):
    """Comparator written for these tests: the full logits rounded to h's dtype (the library GEMM's output), capped
    in fp32, the exact softmax from their log-sum-exp, the softmax terms rounded to h's dtype before they meet W (the
    reference's p.to(h.dtype) @ W). Targets outside [0, V) contribute no target logit and no target row."""
    V = W.shape[0]
    z = (h @ W.t()).float()
    dz = torch.ones_like(z)
    if softcap:
        t = torch.tanh(z / softcap)
        z, dz = softcap * t, 1 - t * t
    lse = torch.logsumexp(z, -1)
    ok = (tgt >= 0) & (tgt < V)
    idx = torch.where(ok, tgt, torch.zeros_like(tgt))
    zt = torch.where(ok, z.gather(1, idx[:, None])[:, 0], torch.zeros_like(lse))
    p = torch.exp(z - lse[:, None])
    p[torch.arange(len(tgt), device=h.device)[ok], idx[ok]] -= 1.0
    g = ((p * dz).to(h.dtype) @ W).float()
    return (lse - zt).sum(), g


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("softcap", [0.0, 30.0])
def test_split_k_gradient_chunks(lm, dtype, softcap):
    """Vocabulary chunks of 4096 columns take the 8-slice split-K gradient GEMM ([parts][n][vc/parts] softmax terms,
    per-slice products summed in fixed order by smel_ce_acc_update); the last chunk (100 columns) falls back to one
    slice. Loss and gradient against the fp64 full-logit oracle and the rounded full-logit comparator."""
    loss_mod, _ = lm
    print(f"split-K CE {dtype} softcap {softcap}", flush=True)
    torch.manual_seed(4)
    n, H, V = 300, 256, 2 * 4096 + 100
    h = (torch.randn(n, H, device="cuda") * 0.5).to(dtype)
    W = (torch.randn(V, H, device="cuda") * 0.2).to(dtype)
    tgt = torch.randint(0, V, (n,), device="cuda")
    tgt[:4] = torch.tensor([0, 4095, 4096, V - 1])                      # chunk edges and the short last chunk
    head = loss_mod.LMHead(weight=W, vocab_chunk=4096, softcap=softcap)
    assert [loss_mod._split_parts(v1 - v0) for v0, v1 in head.chunks()] == [8, 8, 1]
    l1, g1 = loss_mod._ce_chunk(h, head, tgt, True)
    l64, g64 = LR.full_ce(h, W, tgt, softcap)
    lc, gc = rounded_full_ce(h, W, tgt, softcap)
    tol_l, tol_g = (1e-3, 3e-2) if dtype == torch.bfloat16 else (1e-5, 1e-4)
    assert abs(l1.item() - float(l64)) / abs(float(l64)) < tol_l
    assert (g1.double().cpu() - g64).norm() / g64.norm() < tol_g
    assert abs(l1.item() - lc.item()) / abs(lc.item()) < tol_l
    assert (g1 - gc).norm() / gc.norm() < (2e-2 if dtype == torch.bfloat16 else 1e-4)
    l2, g2 = loss_mod._ce_chunk_two_pass(h, head, tgt, True)           # the same sums without any rescaling
    assert abs(l1.item() - l2.item()) / abs(l2.item()) < tol_l
    assert (g1 - g2).norm() / g2.norm() < (2e-2 if dtype == torch.bfloat16 else 1e-5)


def test_targets_outside_the_vocabulary(lm):
    """A target outside [0, V) (e.g. an ignore index of -100 that a caller did not filter) matches no row: its loss
    term is the log-sum-exp alone and its gradient has no target row, as in the reference's _ce_chunk; no row of W is
    gathered for it."""
    loss_mod, _ = lm
    torch.manual_seed(5)
    n, H, V = 40, 64, 900
    h = torch.randn(n, H, device="cuda") * 0.5
    W = torch.randn(V, H, device="cuda") * 0.2
    tgt = torch.randint(0, V, (n,), device="cuda")
    tgt[3], tgt[7], tgt[11] = -100, V, V + 1000
    for softcap in (0.0, 30.0):
        head = loss_mod.LMHead(weight=W, vocab_chunk=256, softcap=softcap)
        l1, g1 = loss_mod._ce_chunk(h, head, tgt, True)
        lc, gc = rounded_full_ce(h, W, tgt, softcap)
        assert abs(l1.item() - lc.item()) < 1e-4 * abs(lc.item())
        assert (g1 - gc).norm() / gc.norm() < 1e-4
