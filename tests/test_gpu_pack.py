"""pack_layer on the GPU (int4 banks from smel_quantize_int4) against the reference's own packed layers
(tests/golden/pack_layer.safetensors, written by the reference's pack_layer, smel/pack.py:8-25): every tensor, name,
order and dtype bit for bit, from a device dict and from a host dict (whose results stay on the host); the LoRA merge
on device tensors; and a packed layer read back by smel.stream.build_layer gives the same MoE layer, forward and
backward, bit for bit, as the layer built from the same quantized bank directly."""
import json
import os

import pytest
import torch
from safetensors import safe_open
from safetensors.torch import load_file

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "pack_layer.safetensors")
SEL = [3, 17]


@pytest.fixture(scope="module")
def mods():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from smel import moe, pack, quant, stream
    return moe, pack, quant, stream


@pytest.fixture(scope="module")
def gold():
    with safe_open(GOLDEN, "pt") as f:
        order = json.loads(f.metadata()["order"])
    g = load_file(GOLDEN)
    t = {k[3:]: v for k, v in g.items() if k.startswith("in.")}
    dense = [k for k in order["nosel"] if not k.startswith("experts.")]
    t = {**{k: t[k] for k in dense}, **{k: v for k, v in t.items() if k not in dense}}
    return g, order, t


def _bits(t):
    return t.view(torch.int16) if t.dtype in (torch.bfloat16, torch.float16) else t


@pytest.mark.parametrize("where", ["cuda", "cpu"])
@pytest.mark.parametrize("tag,ids,group", [("sel", SEL, 64), ("nosel", None, 32)])
def test_pack_layer_golden(mods, gold, where, tag, ids, group):
    _, pack, _, _ = mods
    g, order, t = gold
    print(f"pack_layer {tag} g{group} from {where}", flush=True)
    got = pack.pack_layer({k: v.to(where) for k, v in t.items()}, ids, group)
    assert list(got) == order[tag]
    for k in order[tag]:
        want = g[f"{tag}.{k}"]
        v = got[k]
        assert v.device.type == ("cpu" if k == "experts.sel.ids" else where), k
        assert v.dtype == want.dtype and v.shape == want.shape and v.is_contiguous(), k
        assert torch.equal(_bits(v.cpu()), _bits(want)), k


def test_merge_on_device(mods, gold):
    """merge_experts / merge_mlp on device tensors: the fp32 product B A runs on the GPU's BLAS, whose sums may round
    differently from the host's, so a merged weight may sit one bf16 step from the reference's where the fp32 sum
    lies on a rounding boundary: at most 1 weight in 10^3 and never more than one step."""
    _, pack, _, _ = mods
    from smel.lora import ExpertsLoRA, MLPLoRA
    g, _, t = gold
    ex, sh = ExpertsLoRA(SEL, 64, 64, r=4, alpha=6.0).cuda(), MLPLoRA(64, 96, r=4, alpha=6.0).cuda()
    with torch.no_grad():
        for n in ("A_gate", "A_up", "A_down", "B_gate", "B_up", "B_down"):
            getattr(ex, n).copy_(g["lora.ex_" + n])
            getattr(sh, n).copy_(g["lora.sh_" + n])
    gu, dn = pack.merge_experts(t["mlp.experts.gate_up_proj"].cuda(), t["mlp.experts.down_proj"].cuda(), ex)
    p = "mlp.shared_expert."
    shw = pack.merge_mlp(*(t[p + n + "_proj.weight"].cuda() for n in ("gate", "up", "down")), sh)
    pairs = [(gu[SEL], g["merge.gate_up_sel"]), (dn[SEL], g["merge.down_sel"])]
    pairs += [(w, g["merge.sh_" + n]) for n, w in zip(("gate", "up", "down"), shw)]
    for got, want in pairs:
        d = (_bits(got.cpu()).int() - _bits(want).int()).abs()
        assert d.max() <= 1 and int((d > 0).sum()) <= max(1, want.numel() // 1000)


def test_packed_layer_reads_back(mods):
    """pack_layer -> build_layer (the packed branch) -> moe_forward + backward equals the layer built from the bf16
    checkpoint tensors with the same int4 bank and selection, bit for bit."""
    moe, pack, quant, stream = mods
    H, E, I, K, T = 256, 16, 128, 4, 384
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(5)
    rn = lambda *s: (torch.randn(*s, generator=gen, device=dev) * 0.02).to(torch.bfloat16)
    t = {"mlp.gate.weight": rn(E, H), "mlp.shared_expert.gate_proj.weight": rn(I, H),
         "mlp.shared_expert.up_proj.weight": rn(I, H), "mlp.shared_expert.down_proj.weight": rn(H, I),
         "mlp.shared_expert_gate.weight": rn(1, H), "mlp.experts.gate_up_proj": rn(E, 2 * I, H),
         "mlp.experts.down_proj": rn(E, H, I)}
    sel = [2, 9, 11]
    LWp = stream.build_layer(0, "linear_attention", pack.pack_layer(t, sel, 64))
    bank = moe.Int4Experts(quant.quantize_int4(t["mlp.experts.gate_up_proj"], 64),
                           quant.quantize_int4(t["mlp.experts.down_proj"], 64), dtype=torch.bfloat16)
    ids = torch.tensor(sel, device=dev)
    ex = moe.LayerExperts(bank, sel, t["mlp.experts.gate_up_proj"][ids], t["mlp.experts.down_proj"][ids])
    LWd = stream.LayerWeights(0, "linear_attention", {k: v for k, v in t.items() if not k.startswith("mlp.experts")},
                              ex)
    assert LWp.experts.sel_ids.tolist() == sel
    x = torch.randn(T, H, generator=gen, device=dev).to(torch.bfloat16)
    gy = (torch.randn(T, H, generator=gen, device=dev) * 1e-3).to(torch.bfloat16)
    outs = []
    for LW in (LWp, LWd):
        xg = x.clone().requires_grad_(True)
        y = moe.moe_forward(xg, LW.W, LW.experts, K)
        y.backward(gy)
        outs.append((y.detach(), xg.grad))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
