"""The LoRA containers and dense helpers of smel.lora against the adapter format and formulas of the reference's
smel/lora.py (CPU only): parameter names, order, shapes and dtypes; the init (A uniform in +-1/sqrt(in), B zero);
delta = scale B A; lora_linear / lora_gate_up against the plain fp64 formula x w^T + s (x A^T) B^T and its
gradients; an adapter folder written in the reference trainer's format loads back bit for bit."""
import json
import math
import os

import torch

from smel.lora import BlockLoRA, ExpertsLoRA, LayerLoRA, MLPLoRA, lora_gate_up, lora_linear

NAMES = ["A_gate", "B_gate", "A_up", "B_up", "A_down", "B_down"]


def test_parameter_format():
    torch.manual_seed(0)
    ex = ExpertsLoRA([3, 9, 40], hidden=64, inter=32, r=4, alpha=8.0)
    sh = MLPLoRA(64, 48, r=4, alpha=8.0)
    assert [n for n, _ in ex.named_parameters()] == NAMES and [n for n, _ in sh.named_parameters()] == NAMES
    assert ex.expert_ids.tolist() == [3, 9, 40] and "expert_ids" in ex.state_dict()
    shapes = {"A_gate": (3, 4, 64), "B_gate": (3, 32, 4), "A_up": (3, 4, 64), "B_up": (3, 32, 4),
              "A_down": (3, 4, 32), "B_down": (3, 64, 4)}
    for n, s in shapes.items():
        p = getattr(ex, n)
        assert tuple(p.shape) == s and p.dtype == torch.float32 and p.requires_grad
    assert tuple(sh.A_down.shape) == (4, 48) and tuple(sh.B_down.shape) == (64, 4)
    assert ex.scale == 2.0 and sh.r == 4 and sh.alpha == 8.0
    for m in (ex, sh):
        for n in ("B_gate", "B_up", "B_down"):
            assert not getattr(m, n).any()


def test_init_is_kaiming_uniform_sqrt5():
    """Bound 1/sqrt(in) and the uniform distribution's moments (mean 0, variance bound^2 / 3) per factor, and the
    same bound as torch's kaiming_uniform_(a=sqrt(5)) reports through its own formula."""
    torch.manual_seed(1)
    ex = ExpertsLoRA(list(range(8)), hidden=2048, inter=512, r=16)
    for n, fan in (("A_gate", 2048), ("A_up", 2048), ("A_down", 512)):
        a = getattr(ex, n).detach()
        b = 1.0 / math.sqrt(fan)
        gain = torch.nn.init.calculate_gain("leaky_relu", math.sqrt(5))
        assert abs(gain * math.sqrt(3.0 / fan) - b) < 1e-12
        assert a.abs().max() <= b and a.abs().max() > 0.99 * b
        assert abs(a.mean().item()) < 0.01 * b and abs(a.var().item() / (b * b / 3) - 1) < 0.02
        # every expert's matrices are drawn separately (no two slots equal)
        assert not torch.equal(a[0], a[1])


def test_delta():
    torch.manual_seed(2)
    ex = ExpertsLoRA([1, 5], 16, 8, r=2, alpha=6.0)
    with torch.no_grad():
        for n in ("B_gate", "B_up", "B_down"):
            getattr(ex, n).normal_()
    dg, du, dd = ex.delta(1)
    assert torch.allclose(dg, 3.0 * ex.B_gate[1] @ ex.A_gate[1]) and dd.shape == (16, 8)
    assert torch.allclose(du, 3.0 * ex.B_up[1] @ ex.A_up[1])
    sh = MLPLoRA(16, 8, r=2, alpha=2.0)
    with torch.no_grad():
        sh.B_down.normal_()
    assert torch.allclose(sh.delta()[2], sh.B_down @ sh.A_down)


def _plain(x, w, A, B, s):
    return x @ w.t() + s * ((x @ A.t()) @ B.t())


def test_dense_helpers_match_plain_formula():
    torch.manual_seed(3)
    T, H, I, r, s = 11, 24, 10, 3, 1.5
    x = torch.randn(T, H, dtype=torch.float64, requires_grad=True)
    wgu = torch.randn(2 * I, H, dtype=torch.float64)
    fac = {n: torch.randn(*shp, dtype=torch.float64, requires_grad=True)
           for n, shp in (("A_gate", (r, H)), ("B_gate", (I, r)), ("A_up", (r, H)), ("B_up", (I, r)))}
    g, u = lora_gate_up(x, wgu, fac["A_gate"], fac["B_gate"], fac["A_up"], fac["B_up"], s)
    gp = _plain(x, wgu[:I], fac["A_gate"], fac["B_gate"], s)
    up = _plain(x, wgu[I:], fac["A_up"], fac["B_up"], s)
    assert torch.allclose(g, gp, atol=1e-12) and torch.allclose(u, up, atol=1e-12)
    cot = torch.randn(T, 2 * I, dtype=torch.float64)
    got = torch.autograd.grad((torch.cat((g, u), 1) * cot).sum(), [x, *fac.values()])
    want = torch.autograd.grad((torch.cat((gp, up), 1) * cot).sum(), [x, *fac.values()])
    for a, b in zip(got, want):
        assert torch.allclose(a, b, atol=1e-10)
    g0, u0 = lora_gate_up(x, wgu, None, None, None, None, s)
    assert torch.allclose(torch.cat((g0, u0), 1), x @ wgu.t())
    wd = torch.randn(H, I, dtype=torch.float64)
    A, B = torch.randn(r, I, dtype=torch.float64), torch.randn(H, r, dtype=torch.float64)
    a = torch.randn(T, I, dtype=torch.float64)
    assert torch.allclose(lora_linear(a, wd, A, B, s), _plain(a, wd, A, B, s), atol=1e-12)
    assert torch.allclose(lora_linear(a, wd, None, None, s), a @ wd.t())
    # 3-D activations and bf16 rows: factors cast to the rows' dtype
    xb = torch.randn(2, 5, H).bfloat16()
    yb = lora_linear(xb, wgu.bfloat16(), fac["A_gate"].detach().float(), torch.randn(2 * I, r), s)
    assert yb.dtype == torch.bfloat16 and yb.shape == (2, 5, 2 * I)


def test_dense_helpers_bf16_round_once():
    """bf16 rows as a matrix: the scaled LoRA term is added in the second LoRA product's epilogue (torch.addmm with
    alpha, smel/lora.py:61-83), so it is not rounded on its own before the add. Bitwise equal to that form for both
    helpers, and different from rounding the LoRA product first (so the check can fail)."""
    torch.manual_seed(5)
    T, H, I, r, s = 64, 96, 40, 8, 2.0
    bf = torch.bfloat16
    x = torch.randn(T, H).to(bf)
    wgu = (torch.randn(2 * I, H) * 0.1).to(bf)
    Ag, Au = torch.randn(r, H) * 0.1, torch.randn(r, H) * 0.1
    Bg, Bu = torch.randn(I, r) * 0.1, torch.randn(I, r) * 0.1
    g, u = lora_gate_up(x, wgu, Ag, Bg, Au, Bu, s)
    base = x @ wgu.t()
    xa = x @ torch.cat((Ag, Au)).to(bf).t()
    g_ref = torch.addmm(base[:, :I], xa[:, :r], Bg.to(bf).t(), alpha=s)
    u_ref = torch.addmm(base[:, I:], xa[:, r:], Bu.to(bf).t(), alpha=s)
    assert torch.equal(g, g_ref) and torch.equal(u, u_ref)
    y = lora_linear(x, wgu[:I], Ag, Bg, s)
    y_ref = torch.addmm(x @ wgu[:I].t(), x @ Ag.to(bf).t(), Bg.to(bf).t(), alpha=s)
    assert torch.equal(y, y_ref)
    twice = torch.add(x @ wgu[:I].t(), (x @ Ag.to(bf).t()) @ Bg.to(bf).t(), alpha=s)
    assert not torch.equal(y, twice)
    # rows of a leading shape: the same values as the flattened matrix
    g3, u3 = lora_gate_up(x.reshape(4, 16, H), wgu, Ag, Bg, Au, Bu, s)
    assert torch.equal(g3.reshape(T, I), g) and torch.equal(u3.reshape(T, I), u)


def test_block_build_and_adapter_roundtrip(tmp_path):
    """BlockLoRA.build over a selection, then an adapter folder in the reference trainer's format (config keys
    experts / r / alpha / shared_lora, tensors under the module paths) loads back equal."""
    from safetensors.torch import save_file

    class Dims:
        hidden, moe_inter, shared_inter = 32, 16, 24

    torch.manual_seed(4)
    sel = {3: [0, 7], 5: [], 9: [2]}
    blk = BlockLoRA.build(sel, 32, 16, 24, r=4, alpha=8.0)
    assert blk.get(5).experts is None and isinstance(blk.get(5).shared, MLPLoRA) and blk.get(4) is None
    assert blk.get(3).experts.expert_ids.tolist() == [0, 7] and isinstance(blk.get(9), LayerLoRA)
    with torch.no_grad():
        for p in blk.parameters():
            p.normal_()
    os.makedirs(tmp_path / "ad")
    save_file({k: v.contiguous() for k, v in blk.state_dict().items()}, str(tmp_path / "ad" / "adapter.safetensors"))
    with open(tmp_path / "ad" / "adapter_config.json", "w") as f:
        json.dump({"experts": {str(k): v for k, v in sel.items()}, "r": 4, "alpha": 8.0, "shared_lora": True}, f)
    back, meta = BlockLoRA.load(str(tmp_path / "ad"), Dims, device="cpu")
    assert meta["r"] == 4
    sd0, sd1 = blk.state_dict(), back.state_dict()
    assert list(sd0) == list(sd1)
    for k in sd0:
        assert torch.equal(sd0[k], sd1[k]), k
    assert BlockLoRA.build({1: [0]}, 32, 16, 24, r=4, alpha=8.0, shared=False).get(1).shared is None
