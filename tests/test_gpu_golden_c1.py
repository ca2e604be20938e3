"""The HIP layer on the reference's own C1 vectors (tests/golden/c1_moe_fp32.safetensors, written by the reference's
smel/moe.py moe_forward on its fp32 CPU path, tests/test_moe.py:10-36's setting): y, dX and all twelve LoRA
gradients against the golden outputs at the bf16 bar.

The golden routing is forced: the router formula of smel/moe.py:162-167 (fp32 softmax of x Wr^T, the golden ids,
renormalised, rounded to the logits' dtype) runs as torch ops on the bf16 inputs with the golden ids, and the layer
is composed as the reference composes it (smel/moe.py:255-263: routed_experts + shared_mlp), both on the HIP kernels.
The fused moe_forward routes by itself; tokens are independent in y and dX, so it is compared on every token whose
own top-k ids equal the golden ones."""
import pytest
import torch

from helpers import LORA_NAMES, assert_close_bf16, c1_layer, to_device_layer

pytestmark = pytest.mark.gpu
DEV = "cuda"
K = 2


def _say(msg):
    print(msg, flush=True)


def _inputs(t):
    W, ex, lora = to_device_layer(c1_layer(t), DEV)
    x = t["in.x"].to(DEV, torch.bfloat16)
    gy = t["in.gy"].to(DEV, torch.bfloat16)
    return W, ex, lora, x, gy


def _forced_topv(x, gate_w, topi):
    """The reference's route (smel/moe.py:162-167) with the ids given: fp32 softmax over x Wr^T, the given ids'
    probabilities renormalised and rounded to the logits' dtype; differentiable w.r.t. x."""
    logits = (x @ gate_w.t()).float()
    probs = torch.softmax(logits, dim=-1)
    tv = probs.gather(1, topi)
    return (tv / tv.sum(-1, keepdim=True)).to(x.dtype)


def test_c1_golden_forced_routing(golden_c1):
    """routed_experts + shared_mlp on the HIP kernels with the golden routing: y, dX and every LoRA gradient of both
    sets against the reference's golden values."""
    from smel.moe import routed_experts, shared_mlp
    _say("C1 golden, forced routing")
    t = golden_c1
    W, ex, lora, x, gy = _inputs(t)
    topi = t["out.topi"].to(DEV)
    xg = x.clone().requires_grad_(True)
    topv = _forced_topv(xg, W["mlp.gate.weight"], topi)
    y = routed_experts(xg, topv, topi, ex, lora.experts) + shared_mlp(xg, W, lora.shared)
    y.backward(gy)
    torch.cuda.synchronize()
    e, m, c = assert_close_bf16(y.detach().cpu(), t["out.y"], "y")
    _say(f"  y: rel {e:.2e} max {m:.2e} cos {c:.7f}")
    e, m, c = assert_close_bf16(xg.grad.cpu(), t["out.dx"], "dx")
    _say(f"  dx: rel {e:.2e} max {m:.2e} cos {c:.7f}")
    for tag, mod in (("ex", lora.experts), ("sh", lora.shared)):
        for n in LORA_NAMES:
            e, m, c = assert_close_bf16(getattr(mod, n).grad.cpu(), t[f"out.d_{tag}_{n}"], f"d_{tag}_{n}")
            _say(f"  d_{tag}_{n}: rel {e:.2e} max {m:.2e} cos {c:.7f}")


def test_c1_golden_routed_only(golden_c1):
    """routed_experts alone (no grad) equals the reference's routed part for the golden routing."""
    from smel.moe import routed_experts
    t = golden_c1
    W, ex, lora, x, _ = _inputs(t)
    topi = t["out.topi"].to(DEV)
    with torch.no_grad():
        out = routed_experts(x, t["out.topv"].to(DEV, torch.bfloat16), topi, ex, lora.experts)
    assert_close_bf16(out.cpu(), t["out.routed"], "routed")


def _same_route_rows(topi, golden_topi):
    """Tokens whose top-k ids (as sets) equal the golden ones."""
    a, b = topi.cpu().sort(-1).values, golden_topi.sort(-1).values
    return (a == b).all(-1)


@pytest.mark.parametrize("with_sel", [True, False])
def test_c1_golden_fused_layer(golden_c1, with_sel):
    """moe_forward (router, dispatch, expert GEMMs, combine, shared expert and their backward fused): y and dX on the
    tokens the HIP router routes as the reference did (at least 90 % of them; all 128 on this fixture), with and
    without selected experts and LoRA (the golden frozen-only layer); when every token is routed as the reference
    did, all twelve LoRA gradients as well."""
    from smel.moe import moe_forward
    _say(f"C1 golden, fused layer (selection: {with_sel})")
    t = golden_c1
    W, ex, lora = to_device_layer(c1_layer(t, with_sel=with_sel), DEV)
    x = t["in.x"].to(DEV, torch.bfloat16).requires_grad_(True)
    seen = {}
    y = moe_forward(x, W, ex, K, lora if with_sel else None, stats=lambda p, v, i: seen.update(i=i.clone()))
    y.backward(t["in.gy"].to(DEV, torch.bfloat16))
    torch.cuda.synchronize()
    keep = _same_route_rows(seen["i"], t["out.topi"])
    _say(f"  tokens routed as the reference: {int(keep.sum())} / {keep.numel()}")
    assert keep.float().mean() >= 0.9
    ky, kdx = ("out.y", "out.dx") if with_sel else ("out.y_frozen_only", "out.dx_frozen_only")
    e, m, c = assert_close_bf16(y.detach().cpu()[keep], t[ky][keep], "y")
    _say(f"  y: rel {e:.2e} max {m:.2e} cos {c:.7f}")
    e, m, c = assert_close_bf16(x.grad.cpu()[keep], t[kdx][keep], "dx")
    _say(f"  dx: rel {e:.2e} max {m:.2e} cos {c:.7f}")
    if with_sel and bool(keep.all()):   # every token routed as the reference: the LoRA gradients are comparable
        for tag, mod in (("ex", lora.experts), ("sh", lora.shared)):
            for n in LORA_NAMES:
                e, m, c = assert_close_bf16(getattr(mod, n).grad.cpu(), t[f"out.d_{tag}_{n}"], f"d_{tag}_{n}")
                _say(f"  d_{tag}_{n}: rel {e:.2e} max {m:.2e} cos {c:.7f}")
