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
def test_several_vocabulary_chunks(lm, dtype, softcap):
    """Vocabulary chunks of 4096 columns (16 logits tiles, 32 statistics windows) and a short last chunk of 100
    columns (one partly filled tile): the running maximum moves between chunks, so the accumulator and the window
    shifts are rescaled. Loss and gradient against the fp64 full-logit oracle and the rounded full-logit comparator."""
    loss_mod, _ = lm
    print(f"multi-chunk CE {dtype} softcap {softcap}", flush=True)
    torch.manual_seed(4)
    n, H, V = 300, 256, 2 * 4096 + 100
    h = (torch.randn(n, H, device="cuda") * 0.5).to(dtype)
    W = (torch.randn(V, H, device="cuda") * 0.2).to(dtype)
    tgt = torch.randint(0, V, (n,), device="cuda")
    tgt[:6] = torch.tensor([0, 127, 128, 4095, 4096, V - 1])           # window, tile, chunk edges, the last column
    head = loss_mod.LMHead(weight=W, vocab_chunk=4096, softcap=softcap)
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


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_wide_logit_range(lm, dtype):
    """Head rows of very different norms: windows whose maxima lie 100-400 below the row's maximum get shifts past
    the bf16 / fp32 range (their terms become zero, as exp underflows in the reference), others small shifts; a few
    rows put their target in such a window (a large loss). bf16 against the rounded full-logit comparator (logits of
    a few hundred carry bf16 steps of 0.5-2 in both), fp32 against the fp64 oracle."""
    loss_mod, _ = lm
    print(f"wide-range CE {dtype}", flush=True)
    torch.manual_seed(6)
    n, H, V = 96, 128, 3000
    h = torch.randn(n, H, device="cuda").to(dtype)
    scale = torch.ones(V, 1, device="cuda")
    scale[0:128] = 40.0            # window 0: logits of a few hundred
    scale[1024:1152] = 8.0         # a window at a moderate offset
    W = (torch.randn(V, H, device="cuda") * 0.1 * scale).to(dtype)
    tgt = torch.randint(0, V, (n,), device="cuda")
    tgt[:4] = torch.tensor([5, 1030, 2999, 700])
    head = loss_mod.LMHead(weight=W, vocab_chunk=1024)
    l1, g1 = loss_mod._ce_chunk(h, head, tgt, True)
    if dtype == torch.bfloat16:
        lc, gc = rounded_full_ce(h, W, tgt, 0.0)
        assert abs(l1.item() - lc.item()) / abs(lc.item()) < 1e-4
        assert (g1 - gc).norm() / gc.norm() < 2e-2
    else:
        l64, g64 = LR.full_ce(h, W, tgt)
        assert abs(l1.item() - float(l64)) / abs(float(l64)) < 1e-5
        assert (g1.double().cpu() - g64).norm() / g64.norm() < 1e-4


def test_several_row_passes(lm):
    """Passes of 16 rows (a caller's token_chunk bounds the rows of a pass): the loss accumulates over the passes and
    each pass writes its own gradient rows; equal to one pass over all rows."""
    loss_mod, _ = lm
    torch.manual_seed(7)
    n, H, V = 200, 64, 1500
    h = (torch.randn(n, H, device="cuda") * 0.5).bfloat16()
    W = (torch.randn(V, H, device="cuda") * 0.2).bfloat16()
    tgt = torch.randint(0, V, (n,), device="cuda")
    head = loss_mod.LMHead(weight=W, vocab_chunk=512)
    one = h.clone().requires_grad_(True)
    l_one = loss_mod.chunked_ce(one, head, tgt, denom=float(n))
    l_one.backward()
    many = h.clone().requires_grad_(True)
    l_many = loss_mod.chunked_ce(many, head, tgt, denom=float(n), token_chunk=16)
    (l_many * 2.0).backward()                                      # the incoming gradient scales the rows
    assert abs(l_one.item() - l_many.item()) < 1e-5 * abs(l_one.item())
    assert torch.equal(many.grad.float(), (2.0 * one.grad.float()).bfloat16().float())
    l64, g64 = LR.full_ce(h, W, tgt, denom=float(n))
    assert abs(l_many.item() - float(l64)) / abs(float(l64)) < 1e-3


def test_token_chunk_bounds_pass_memory(lm):
    """token_chunk x vocab_chunk bounds a pass's scratch, as the reference promises for its peak memory: with
    token_chunk=256 over 4096 rows, one call allocates at most one 256-row pass (softmax terms 256 x vocab_chunk
    bf16, fp32 row state and accumulators) beyond its gradient output; left at the default, a pass takes all 4096
    rows and its terms alone are 16 times larger. Both give the same loss and gradient."""
    loss_mod, _ = lm
    torch.manual_seed(9)
    n, H, V, vc = 4096, 256, 65536, 32768
    h = torch.randn(n, H, device="cuda").bfloat16()
    W = (torch.randn(V, H, device="cuda") * 0.05).bfloat16()
    tgt = torch.randint(0, V, (n,), device="cuda")
    head = loss_mod.LMHead(weight=W, vocab_chunk=vc)

    def run(**kw):
        x = h.clone().requires_grad_(True)
        loss_mod.chunked_ce(x, head, tgt, denom=float(n), **kw)   # the head's transposed copy is made once, here
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        loss = loss_mod.chunked_ce(x, head, tgt, denom=float(n), **kw)
        loss.backward()
        torch.cuda.synchronize()
        return torch.cuda.max_memory_allocated() - base, loss.detach(), x.grad

    peak_small, l_small, g_small = run(token_chunk=256)
    peak_dflt, l_dflt, g_dflt = run()
    tc = 256
    one_pass = tc * vc * 2 + tc * H * 4 * 3 + 2 * (vc // 128) * tc * 4 + (vc // 128) * tc + 6 * tc * 4
    bound = one_pass + 2 * n * H * 2 + (1 << 20)    # + the gradient output and x.grad (bf16), small tensors
    print(f"CE peak allocation: token_chunk=256 {peak_small / 2**20:.1f} MiB (bound {bound / 2**20:.1f}), default "
          f"{peak_dflt / 2**20:.1f} MiB", flush=True)
    assert peak_small <= bound
    assert peak_dflt > 8 * tc * vc * 2
    # the gradient GEMM splits its contraction by the number of row tiles of a pass, so the two pass sizes sum the
    # fp32 partials in different orders: equal up to the last bits
    assert abs(l_small.item() - l_dflt.item()) <= 1e-5 * abs(l_dflt.item())
    d = (g_small.float() - g_dflt.float()).abs().max().item()
    assert d <= 2**-7 * g_dflt.float().abs().max().item(), d


def test_qwen_head_full_size(lm):
    """The bench's shape (4092 rows, hidden 2048, vocabulary 248320, chunks of 32768, bf16): loss and gradient of
    chunked_ce against the rounded full-logit comparator run in fp32 torch on the GPU (the [4092, 248320] logits fit
    in memory there), and the same call twice gives bitwise equal results."""
    loss_mod, _ = lm
    print("CE full size", flush=True)
    torch.manual_seed(8)
    T, H, V = 4092, 2048, 248320
    h = torch.randn(T, H, device="cuda").bfloat16()
    W = (torch.randn(V, H, device="cuda") * 0.02).bfloat16()
    tgt = torch.randint(0, V, (T,), device="cuda")
    head = loss_mod.LMHead(weight=W)
    x = h.clone().requires_grad_(True)
    loss = loss_mod.chunked_ce(x, head, tgt, denom=float(T))
    loss.backward()
    g1 = x.grad.clone()
    x.grad = None
    loss2 = loss_mod.chunked_ce(x, head, tgt, denom=float(T))
    loss2.backward()
    assert torch.equal(loss, loss2) and torch.equal(g1, x.grad)
    lc, gc = rounded_full_ce(h, W, tgt, 0.0)
    lc, gc = lc / T, gc / T
    rel_l = abs(loss.item() - lc.item()) / abs(lc.item())
    rel_g = ((g1.float() - gc).norm() / gc.norm()).item()
    cos = torch.nn.functional.cosine_similarity(g1.float().flatten(), gc.flatten(), dim=0).item()
    print(f"full-size CE: loss rel err {rel_l:.2e}, grad rel err {rel_g:.2e}, cos {cos:.6f}", flush=True)
    assert rel_l < 1e-4 and rel_g < 2e-2 and cos > 0.9999


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
