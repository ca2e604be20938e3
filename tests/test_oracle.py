"""Pins the CPU oracle: against the reference's own golden vectors (tests/golden, written by the reference code),
against closed forms and brute force, and the C restatement against the numpy one. CPU only."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import LORA_NAMES, QUANT_CASES, c1_layer
from oracle import intref
from oracle import moe_ref as R


# ------------------------------------------------------------------------------------------------------- int4


@pytest.mark.parametrize("case", QUANT_CASES)
def test_quantize_golden(golden_quant, case):
    g = golden_quant
    grp = 32 if case == "g32" else 64
    pk = R.quantize_int4(g[f"quant.{case}.w"], grp)
    assert torch.equal(pk["q"], g[f"quant.{case}.q"])
    assert torch.equal(pk["scale"].view(torch.int16), g[f"quant.{case}.scale"].view(torch.int16))
    assert torch.equal(pk["zero"].view(torch.int16), g[f"quant.{case}.zero"].view(torch.int16))


def test_quantize_rejects_bad_group():
    with pytest.raises(AssertionError):
        R.quantize_int4(torch.randn(2, 48), 64)


@pytest.mark.parametrize("case", QUANT_CASES)
def test_dequant_golden(golden_quant, case):
    g = golden_quant
    q, s, z = g[f"quant.{case}.q"], g[f"quant.{case}.scale"], g[f"quant.{case}.zero"]
    f32 = R.dequant_int4(q, s, z, torch.float32)
    assert torch.equal(f32, g[f"quant.{case}.deq_f32"])
    assert torch.equal(R.dequant_int4_bf16math(q, s, z).view(torch.int16),
                       g[f"quant.{case}.deq_bf16_torch"].view(torch.int16))
    # the GPU-kernel bf16 value is one RNE of the reference's exact fp32 value
    want = g[f"quant.{case}.deq_f32"].to(torch.bfloat16).view(torch.int16)
    assert torch.equal(R.dequant_int4(q, s, z, torch.bfloat16).view(torch.int16), want)
    sb, zb = s.view(torch.int16).numpy().view(np.uint16), z.view(torch.int16).numpy().view(np.uint16)
    np_bits = intref.dequant_bits(q.numpy(), sb, zb)
    c_bits = intref.c_dequant_bits(q.numpy(), sb, zb)
    assert np.array_equal(np_bits, want.numpy().view(np.uint16))
    assert np.array_equal(c_bits, np_bits)
    assert np.array_equal(intref.c_dequant_bits(q.numpy(), sb, zb, out_f32=True),
                          g[f"quant.{case}.deq_f32"].numpy())


def test_int4_grid_roundtrip(golden_quant):
    """smel tests/test_quant_merge.py:14-23: exact-grid weights come back up to bf16 rounding of scale/zero."""
    torch.manual_seed(0)
    q = torch.randint(0, 16, (4, 8, 128))
    scale = (torch.rand(4, 8, 2) + 0.5).bfloat16().float()
    zero = torch.randn(4, 8, 2).bfloat16().float()
    w = (q.reshape(4, 8, 2, 64).float() * scale[..., None] + zero[..., None]).reshape(4, 8, 128)
    pk = R.quantize_int4(w, 64)
    back = R.dequant_int4(pk["q"], pk["scale"], pk["zero"], torch.float32)
    assert R.rel_err(back, w) < 5e-3
    # the fixture's grid case went through the reference quantizer: its dequant is the reference's own
    g = golden_quant
    assert torch.equal(R.dequant_int4(g["quant.grid.q"], g["quant.grid.scale"], g["quant.grid.zero"],
                                      torch.float32), g["quant.grid.deq_f32"])


def test_nibble_order_matters():
    """A swapped nibble order would be caught: the low nibble holds the even column."""
    q = torch.tensor([[0x1F]], dtype=torch.uint8)
    s = torch.ones(1, 1, dtype=torch.bfloat16)
    z = torch.zeros(1, 1, dtype=torch.bfloat16)
    assert R.dequant_int4(q, s, z, torch.float32).tolist() == [[15.0, 1.0]]


def test_bf16_rne_three_ways():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(100000).astype(np.float32) * np.float32(10.0) ** rng.integers(-40, 38, 100000)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9,
                        3.3895314e38, 1e-45, -1e-40], dtype=np.float32)
    x = np.concatenate([x.astype(np.float32), special])
    a = intref.bf16_rne(x)
    b = intref.c_bf16_rne(x)
    c = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    fin = np.isfinite(x)
    assert np.array_equal(a, b)
    assert np.array_equal(a[fin], c[fin])
    assert np.all(np.isnan(intref.bf16_bits_to_f32(a[np.isnan(x)])))
    # ties to even: 1 + 2^-8 is halfway between bf16 1.0 and 1.0078125 -> 1.0
    assert intref.bf16_rne(np.array([1.0 + 2 ** -8], np.float32))[0] == 0x3F80


# ------------------------------------------------------------------------------------------------------ top-k


def test_topk_matches_torch_without_ties():
    g = torch.Generator().manual_seed(0)
    p = torch.softmax(torch.randn(500, 256, generator=g), -1)
    v, i = R.topk_lowest_index(p, 8)
    tv, ti = torch.topk(p, 8)
    assert torch.equal(i, ti) and torch.equal(v, tv)
    cv, ci = intref.c_topk(p.numpy(), 8)
    nv, ni = intref.topk(p.numpy(), 8)
    assert np.array_equal(ci, i.numpy()) and np.array_equal(ni, i.numpy())


def test_topk_ties_lowest_index_first():
    g = torch.Generator().manual_seed(1)
    p = torch.randint(0, 5, (300, 64), generator=g).float()
    v, i = R.topk_lowest_index(p, 8)
    for r in range(p.shape[0]):
        want = sorted(range(64), key=lambda c: (-p[r, c].item(), c))[:8]
        assert i[r].tolist() == want
    ci = intref.c_topk(p.numpy(), 8)[1]
    assert np.array_equal(ci, i.numpy())
    # the value set always agrees with torch.topk
    tv, _ = torch.topk(p, 8)
    assert torch.equal(tv, v)


# --------------------------------------------------------------------------------------------------- dispatch


@pytest.mark.parametrize("T,K,E", [(128, 2, 8), (333, 8, 256), (1, 8, 256), (0, 8, 16), (64, 4, 3)])
def test_dispatch_three_ways(T, K, E):
    g = torch.Generator().manual_seed(T + K + E)
    if E >= K:
        topi = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]) if T else \
            torch.zeros(0, K, dtype=torch.long)
    else:
        topi = torch.randint(0, E, (T, K), generator=g)
    order, tok, counts, offsets, inv = R.dispatch(topi, E)
    o2, t2, c2, off2, i2 = R.dispatch_fast(topi, E)
    assert torch.equal(order, o2) and torch.equal(counts, c2) and torch.equal(inv, i2)
    nc, noff, nord, ninv = intref.dispatch(topi.numpy(), E)
    cc, coff, cord, cinv = intref.c_dispatch(topi.numpy(), E)
    for a, b in ((nc, cc), (noff, coff), (nord, cord), (ninv, cinv)):
        assert np.array_equal(a, b)
    assert np.array_equal(nord, order.numpy())
    # invariants: permutation, sum of counts, offsets = exclusive cumsum, p ascending within an expert
    flat = topi.reshape(-1)
    assert sorted(order.tolist()) == list(range(T * K))
    assert int(counts.sum()) == T * K and offsets[-1] == T * K
    for e in range(E):
        seg = order[offsets[e]:offsets[e + 1]]
        assert bool((flat[seg] == e).all())
        assert bool((seg[1:] > seg[:-1]).all())
    assert torch.equal(order[inv], torch.arange(T * K))


def test_dispatch_rejects_bad_ids():
    with pytest.raises(ValueError):
        intref.c_dispatch(np.array([[0, 9]]), 8)


# ------------------------------------------------------------------------------------------- act / LoRA


@pytest.mark.parametrize("name", ["silu", "gelu_tanh"])
def test_act_grad(name):
    g = torch.randn(200, dtype=torch.float64, requires_grad=True)
    a, da = R.act_and_grad(g.detach(), name)
    ref = F.silu(g) if name == "silu" else F.gelu(g, approximate="tanh")
    assert torch.allclose(a, ref.detach())
    (auto,) = torch.autograd.grad(ref.sum(), g)
    assert torch.allclose(da, auto)
    assert torch.autograd.gradcheck(lambda t: R.act(t, name), (g[:20].detach().clone().requires_grad_(True),))
    with pytest.raises(ValueError):
        R.act(g, "relu")


def test_lora_plain_formula():
    """smel tests/test_lora_fused.py:13-29 in fp64, including all gradients."""
    torch.manual_seed(0)
    T, H, I, r, s = 33, 64, 48, 4, 2.0
    x = torch.randn(T, H, dtype=torch.float64, requires_grad=True)
    wgu = torch.randn(2 * I, H, dtype=torch.float64)
    P = [torch.randn(*sh, dtype=torch.float64, requires_grad=True) for sh in ((r, H), (I, r), (r, H), (I, r))]

    def plain(w, A, B):
        return x @ w.t() + s * ((x @ A.t()) @ B.t())

    g, u = R.lora_gate_up(x, wgu, *P, s)
    gr, ur = plain(wgu[:I], P[0], P[1]), plain(wgu[I:], P[2], P[3])
    assert torch.allclose(g, gr) and torch.allclose(u, ur)
    assert torch.allclose(R.lora_linear(x, wgu[:I], P[0], P[1], s), gr)
    cot = torch.randn(T, I, dtype=torch.float64)
    ga = torch.autograd.grad((g * cot).sum() + (u * cot).sum(), [x] + P)
    gb = torch.autograd.grad((gr * cot).sum() + (ur * cot).sum(), [x] + P)
    assert all(torch.allclose(a, b) for a, b in zip(ga, gb))


# ------------------------------------------------------------------------------------------ C1 end to end


def test_route_golden(golden_c1):
    t = golden_c1
    probs, topv, topi = R.route(t["in.x"], t["in.gate_w"], 2)
    assert torch.equal(topi, t["out.topi"])
    assert torch.allclose(probs, t["out.probs"], rtol=1e-6, atol=1e-7)
    assert torch.allclose(topv, t["out.topv"], rtol=1e-6, atol=1e-7)


def test_route_gemma4_golden(golden_c1):
    t = golden_c1
    W = {k[len("gemma."):]: v for k, v in t.items() if k.startswith("gemma.router")}
    probs, topv, topi = R.route_gemma4(t["in.x"], W, 2, 1e-6)
    assert torch.equal(topi, t["gemma.topi"])
    assert torch.allclose(probs, t["gemma.probs"], rtol=1e-6, atol=1e-7)
    assert torch.allclose(topv, t["gemma.topv"], rtol=1e-6, atol=1e-7)


def test_dequant_bank_golden(golden_c1):
    t = golden_c1
    L = c1_layer(t)
    gu, dn = L.frozen_weights(0, 8, torch.float32)
    assert torch.equal(gu, t["out.deq_gate_up"]) and torch.equal(dn, t["out.deq_down"])


def test_routed_golden(golden_c1):
    t = golden_c1
    L = c1_layer(t)
    y = R.routed_experts(t["in.x"], t["out.topv"], t["out.topi"], L, L.ex_lora)
    assert R.rel_err(y, t["out.routed"]) < 1e-6


@pytest.mark.parametrize("with_sel", [True, False])
def test_moe_golden(golden_c1, with_sel):
    t = golden_c1
    L = c1_layer(t, with_sel)
    y, dx, grads = R.moe_forward_backward(t["in.x"], L, 2, t["in.gy"], dtype=torch.float32)
    if with_sel:
        assert R.rel_err(y, t["out.y"]) < 1e-6
        assert R.rel_err(dx, t["out.dx"]) < 1e-6
        for tag in ("ex", "sh"):
            for n in LORA_NAMES:
                assert R.rel_err(grads[f"{tag}_{n}"], t[f"out.d_{tag}_{n}"]) < 1e-5, (tag, n)
    else:
        assert R.rel_err(y, t["out.y_frozen_only"]) < 1e-6
        assert R.rel_err(dx, t["out.dx_frozen_only"]) < 1e-6


def test_moe_bruteforce(golden_c1):
    """The composite (dispatch, expert groups, combine) against per-token evaluation, fp64, same routing."""
    t = golden_c1
    L = c1_layer(t)
    x = t["in.x"].double()
    y = R.moe_forward(x, L, 2, forced_topi=t["out.topi"], dtype=torch.float64)
    yb = R.moe_forward_bruteforce(x, L, t["out.topi"], torch.float64)
    assert R.rel_err(y, yb) < 1e-12


def test_moe_stats_hook_and_forced_routes(golden_c1):
    t = golden_c1
    L = c1_layer(t)
    seen = {}

    def stats(p, v, i):
        seen.update(p=p, v=v, i=i)

    R.moe_forward(t["in.x"], L, 2, stats=stats)
    assert torch.equal(seen["i"], t["out.topi"])
    forced = torch.stack([torch.randperm(8)[:2] for _ in range(128)])
    R.moe_forward(t["in.x"], L, 2, stats=stats, forced_topi=forced)
    assert torch.equal(seen["i"], forced)
    assert torch.allclose(seen["v"].sum(-1), torch.ones(128))


def _tiny_gemma(seed=3):
    """A tiny Gemma-4-style block: 8 GELU-tanh experts (2 selected with LoRA), a dense GeGLU MLP with LoRA, router
    tensors as smel/tiny.py:74-77 draws them, plain-weight norms, a layer scalar."""
    T, H, E, I, K, Is, r = 24, 64, 8, 32, 2, 48, 4
    x, L = R.make_layer(T=T, H=H, E=E, I=I, K=K, n_sel=2, r=r, alpha=8.0, shared_inter=None, group=32, seed=seed,
                        act_name="gelu_tanh", lora_b_std=0.05)
    g = torch.Generator().manual_seed(seed + 1)
    rn = lambda *s, std=1.0: torch.randn(*s, generator=g) * std
    W = {f"{n}.weight": (1.0 + 0.2 * rn(H)).to(torch.bfloat16) for n in R.GEMMA4_NORMS}
    W.update({"router.scale": (1.0 + 0.2 * rn(H)).to(torch.bfloat16),
              "router.proj.weight": rn(E, H, std=0.3).to(torch.bfloat16),
              "router.per_expert_scale": (0.5 + torch.rand(E, generator=g)).to(torch.bfloat16),
              "mlp.gate_up_proj.weight": rn(2 * Is, H, std=0.1).to(torch.bfloat16),
              "mlp.down_proj.weight": rn(H, Is, std=0.1).to(torch.bfloat16),
              "layer_scalar": torch.tensor([0.75], dtype=torch.bfloat16)})
    L.sh_lora = {"A_gate": rn(r, H, std=0.1), "A_up": rn(r, H, std=0.1), "A_down": rn(r, Is, std=0.1),
                 "B_gate": rn(Is, r, std=0.1), "B_up": rn(Is, r, std=0.1), "B_down": rn(H, r, std=0.1)}
    L.sh_scale = 2.0
    h = (rn(T, H) * 3.0).to(torch.bfloat16)
    return h, x, W, L, K


def _gemma_block_bruteforce(h, a, W, L, topi, eps):
    """Token by token and slot by slot from the formulas of smel/layer_runner.py:243-262, fp64 throughout."""
    d = lambda t: t.double()
    norm = lambda v, w: v / torch.sqrt((v * v).mean() + eps) * d(w)
    gelu = lambda v: 0.5 * v * (1 + torch.tanh(math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3)))
    gu_all, dn_all = L.frozen_weights(0, L.E, torch.float64)
    sel = {int(e): j for j, e in enumerate(L.sel_ids)}
    S = {k: d(v) for k, v in L.sh_lora.items()}
    Wgu, Wd = d(W["mlp.gate_up_proj.weight"]), d(W["mlp.down_proj.weight"])
    Is = Wd.shape[1]
    H = h.shape[1]
    out = []
    for t in range(h.shape[0]):
        h2 = d(h[t]) + norm(d(a[t]), W["post_attention_layernorm.weight"])
        xm = norm(h2, W["pre_feedforward_layernorm.weight"])
        g = Wgu[:Is] @ xm + L.sh_scale * S["B_gate"] @ (S["A_gate"] @ xm)
        u = Wgu[Is:] @ xm + L.sh_scale * S["B_up"] @ (S["A_up"] @ xm)
        act = gelu(g) * u
        m = norm(Wd @ act + L.sh_scale * S["B_down"] @ (S["A_down"] @ act), W["post_feedforward_layernorm_1.weight"])
        rx = h2 / torch.sqrt((h2 * h2).mean() + eps) * d(W["router.scale"]) * H ** -0.5
        p = torch.softmax(d(W["router.proj.weight"]) @ rx, -1)
        ids = topi[t].tolist()
        v = p[ids] / p[ids].sum() * d(W["router.per_expert_scale"])[ids]
        xe = norm(h2, W["pre_feedforward_layernorm_2.weight"])
        e = torch.zeros(H, dtype=torch.float64)
        for k, ei in enumerate(ids):
            if ei in sel:
                j = sel[ei]
                X = {n: d(L.ex_lora[n][j]) for n in L.ex_lora}
                gu, dn = d(L.sel_gate_up[j]), d(L.sel_down[j])
                I = dn.shape[1]
                ge = gu[:I] @ xe + L.ex_scale * X["B_gate"] @ (X["A_gate"] @ xe)
                ue = gu[I:] @ xe + L.ex_scale * X["B_up"] @ (X["A_up"] @ xe)
                ae = gelu(ge) * ue
                y = dn @ ae + L.ex_scale * X["B_down"] @ (X["A_down"] @ ae)
            else:
                I = dn_all.shape[2]
                ge, ue = gu_all[ei][:I] @ xe, gu_all[ei][I:] @ xe
                y = dn_all[ei] @ (gelu(ge) * ue)
            e += v[k] * y
        e = norm(e, W["post_feedforward_layernorm_2.weight"])
        out.append((h2 + norm(m + e, W["post_feedforward_layernorm.weight"])) * d(W["layer_scalar"]))
    return torch.stack(out)


def test_gemma4_block():
    """The composed Gemma 4 block against a token-by-token fp64 evaluation of the same formulas (same routing); the
    block's norms compute in fp32 as the reference's torch RMSNorm does, hence 1e-5. A plus-one norm weight (the
    Qwen form) or a router without its per-expert scale is shown to fail the same bound."""
    h, a, W, L, K = _tiny_gemma()
    eps = 1e-6
    out, (probs, topv, topi) = R.gemma4_moe_block(h, a, W, L, K, eps, dtype=torch.float64)
    ref = _gemma_block_bruteforce(h, a, W, L, topi, eps)
    assert R.rel_err(out, ref) < 1e-5
    W2 = dict(W, **{"post_feedforward_layernorm_2.weight": (W["post_feedforward_layernorm_2.weight"].float() + 1)
                    .to(torch.bfloat16)})
    assert R.rel_err(_gemma_block_bruteforce(h, a, W2, L, topi, eps), ref) > 1e-3
    W3 = dict(W, **{"router.per_expert_scale": torch.ones_like(W["router.per_expert_scale"])})
    assert R.rel_err(_gemma_block_bruteforce(h, a, W3, L, topi, eps), ref) > 1e-3
    # forced routing reproduces the free choice, and the fp32 autograd wrapper runs end to end
    out_f, _ = R.gemma4_moe_block(h, a, W, L, K, eps, forced_topi=topi, dtype=torch.float64)
    assert torch.equal(out_f, out)
    gy = torch.randn(out.shape, generator=torch.Generator().manual_seed(0))
    y32, dh, da, grads = R.gemma4_block_forward_backward(h, a, W, L, K, eps, gy, forced_topi=topi)
    assert R.rel_err(y32, ref) < 1e-5 and dh.shape == h.shape and da.shape == a.shape
    assert set(grads) == {f"{t}_{n}" for t in ("ex", "sh") for n in L.ex_lora}
    assert all(float(v.abs().sum()) > 0 for v in grads.values())
