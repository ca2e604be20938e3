"""Write the golden vectors in this folder by running the reference's own CPU code once, in the build container.

The reference is Python; it is read as text everywhere else and never travels to the GPU box. This script is the
one place where it is imported (from REF_ROOT, default /root/reference), and only for what no closed form pins
bit-exactly:

* ``quantize_int4`` (smel/quant.py:14-44): exact q/scale/zero bytes depend on the clip-search tie rule and on the
  fp32 reduction order of the squared error;
* the composite ``moe_forward`` / ``routed_experts`` result and its autograd gradients at the tiny config C1
  (smel/moe.py:214-263), as an end-to-end regression value for the oracle;
* ``pack_layer`` / ``merge_experts`` / ``merge_mlp`` (smel/pack.py:8-45) on a small layer dict: the packed format's
  names, dtypes and bytes, and the merged weights' bits.

Everything is generated on the CPU in fp32 with fixed seeds and stored as safetensors (inputs and outputs, so the
tests never re-run this script). Run:  python tests/golden/make_golden.py [quant] [c1] [pack]  (default: all)
"""
import json
import os
import sys

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))
REF_ROOT = os.environ.get("SMEL_REF_ROOT", "/root/reference")


def _import_reference():
    sys.path.insert(0, REF_ROOT)
    from smel import lora as ref_lora  # noqa: E402
    from smel import moe as ref_moe  # noqa: E402
    from smel import quant as ref_quant  # noqa: E402
    return ref_moe, ref_quant, ref_lora


def _import_reference_pack():
    sys.path.insert(0, REF_ROOT)
    from smel import pack as ref_pack  # noqa: E402
    return ref_pack


def c1_inputs(seed=0):
    """Config C1: T=128, H=64, E=8, I=32, K=2, shared Is=32, 2 selected experts + LoRA r=4 (alpha 8), 6 frozen int4
    (gate_up group 64, down group 32 since I=32 cannot hold a group of 64)."""
    g = torch.Generator().manual_seed(seed)
    T, H, E, I, Is, r = 128, 64, 8, 32, 32, 4
    t = {}
    t["x"] = torch.randn(T, H, generator=g)
    t["gate_w"] = torch.randn(E, H, generator=g) * 0.02
    t["gate_up"] = torch.randn(E, 2 * I, H, generator=g) * 0.02
    t["down"] = torch.randn(E, H, I, generator=g) * 0.02
    t["sh_gate"] = torch.randn(Is, H, generator=g) * 0.02
    t["sh_up"] = torch.randn(Is, H, generator=g) * 0.02
    t["sh_down"] = torch.randn(H, Is, generator=g) * 0.02
    t["sh_gate_w"] = torch.randn(1, H, generator=g) * 0.02
    t["sel_ids"] = torch.tensor([1, 4], dtype=torch.long)
    k = 2
    # LoRA: A ~ U(-1/sqrt(in), 1/sqrt(in)) (the kaiming_uniform(a=sqrt(5)) bound), B ~ N(0, 0.02) so dA != 0
    for name, shape in (("A_gate", (k, r, H)), ("A_up", (k, r, H)), ("A_down", (k, r, I))):
        t["ex_" + name] = (torch.rand(*shape, generator=g) * 2 - 1) / shape[-1] ** 0.5
    for name, shape in (("B_gate", (k, I, r)), ("B_up", (k, I, r)), ("B_down", (k, H, r))):
        t["ex_" + name] = torch.randn(*shape, generator=g) * 0.02
    for name, shape in (("A_gate", (r, H)), ("A_up", (r, H)), ("A_down", (r, Is))):
        t["sh_" + name] = (torch.rand(*shape, generator=g) * 2 - 1) / shape[-1] ** 0.5
    for name, shape in (("B_gate", (Is, r)), ("B_up", (Is, r)), ("B_down", (H, r))):
        t["sh_" + name] = torch.randn(*shape, generator=g) * 0.02
    t["gy"] = torch.randn(T, H, generator=g)
    return t


def quant_cases():
    """Weights for quantize_int4 byte vectors: N(0,0.02) expert-like, heavy-tailed, and an exact grid."""
    g = torch.Generator().manual_seed(7)
    cases = {}
    cases["normal"] = (torch.randn(3, 16, 256, generator=g) * 0.02, 64)
    w = torch.randn(2, 8, 128, generator=g)
    w = w * (1 + 4 * (torch.rand(2, 8, 128, generator=g) > 0.97).float())  # outliers drive the clip search
    cases["outlier"] = (w, 64)
    cases["g32"] = (torch.randn(4, 12, 96, generator=g) * 0.05, 32)
    q = torch.randint(0, 16, (4, 8, 128), generator=g)
    sc = (torch.rand(4, 8, 2, generator=g) + 0.5).bfloat16().float()
    ze = torch.randn(4, 8, 2, generator=g).bfloat16().float()
    cases["grid"] = ((q.reshape(4, 8, 2, 64).float() * sc[..., None] + ze[..., None]).reshape(4, 8, 128), 64)
    # more than 16 experts: the reference quantizes 3-D tensors in slices of 16 experts
    cases["e20"] = (torch.randn(20, 4, 64, generator=g) * 0.02, 64)
    return cases


def pack_inputs(seed=11):
    """One layer's tensors as a checkpoint holds them (names relative to the layer): dense weights in fp32, bf16 and
    fp16, SSM parameters A_log / dt_bias (kept fp32), an int64 buffer, and 20 fused bf16 experts (H=64, I=64, more
    than 16 so the quantizer's 16-expert slices show), plus LoRA factors for the merge (r=4, alpha=6: scale 1.5)."""
    g = torch.Generator().manual_seed(seed)
    H, I, E, Is, r = 64, 64, 20, 96, 4
    t = {"input_layernorm.weight": 1 + 0.1 * torch.randn(H, generator=g),
         "linear_attn.A_log": torch.randn(4, generator=g),
         "linear_attn.dt_bias": torch.randn(4, generator=g),
         "linear_attn.in_proj.weight": (torch.randn(3 * H, H, generator=g) * 0.02).bfloat16(),
         "mlp.gate.weight": torch.randn(E, H, generator=g) * 0.02,
         "mlp.shared_expert.gate_proj.weight": (torch.randn(Is, H, generator=g) * 0.02).bfloat16(),
         "mlp.shared_expert.up_proj.weight": (torch.randn(Is, H, generator=g) * 0.02).bfloat16(),
         "mlp.shared_expert.down_proj.weight": (torch.randn(H, Is, generator=g) * 0.02).bfloat16(),
         "mlp.shared_expert_gate.weight": (torch.randn(1, H, generator=g) * 0.02).half(),
         "conv1d.position_ids": torch.arange(7, dtype=torch.int64),
         "mlp.experts.gate_up_proj": (torch.randn(E, 2 * I, H, generator=g) * 0.02).bfloat16(),
         "mlp.experts.down_proj": (torch.randn(E, H, I, generator=g) * 0.02).bfloat16()}
    lo = {}
    for pre, lead, inter in (("ex_", (2,), I), ("sh_", (), Is)):
        for n, shp in (("A_gate", (r, H)), ("A_up", (r, H)), ("A_down", (r, inter))):
            lo[pre + n] = (torch.rand(*lead, *shp, generator=g) * 2 - 1) / shp[-1] ** 0.5
        for n, shp in (("B_gate", (inter, r)), ("B_up", (inter, r)), ("B_down", (H, r))):
            lo[pre + n] = torch.randn(*lead, *shp, generator=g) * 0.05
    return t, lo, [3, 17]


def write_pack():
    ref_pack = _import_reference_pack()
    from smel import lora as ref_lora  # noqa: E402  (already on sys.path)
    t, lo, sel = pack_inputs()
    out = {"in." + k: v.clone() for k, v in t.items()}
    out.update({"lora." + k: v.clone() for k, v in lo.items()})
    order = {}
    for tag, ids, grp in (("sel", sel, 64), ("nosel", None, 32)):
        pk = ref_pack.pack_layer(t, ids, grp)
        order[tag] = list(pk)
        out.update({f"{tag}.{k}": v.clone() for k, v in pk.items()})
    exl = ref_lora.ExpertsLoRA(sel, 64, 64, 4, 6.0)
    shl = ref_lora.MLPLoRA(64, 96, 4, 6.0)
    with torch.no_grad():
        for n in ("A_gate", "A_up", "A_down", "B_gate", "B_up", "B_down"):
            getattr(exl, n).copy_(lo["ex_" + n])
            getattr(shl, n).copy_(lo["sh_" + n])
    gu, dn = ref_pack.merge_experts(t["mlp.experts.gate_up_proj"], t["mlp.experts.down_proj"], exl)
    # only the selected experts' rows change; the other rows equal the input's
    out["merge.gate_up_sel"], out["merge.down_sel"] = gu[sel].clone(), dn[sel].clone()
    assert torch.equal(gu[[e for e in range(20) if e not in sel]],
                       t["mlp.experts.gate_up_proj"][[e for e in range(20) if e not in sel]])
    p = "mlp.shared_expert."
    for n, w in zip(("gate", "up", "down"), ref_pack.merge_mlp(t[p + "gate_proj.weight"], t[p + "up_proj.weight"],
                                                               t[p + "down_proj.weight"], shl)):
        out["merge.sh_" + n] = w
    path = os.path.join(HERE, "pack_layer.safetensors")
    save_file(out, path, metadata={"order": json.dumps(order)})
    os.chmod(path, 0o644)


def main(parts):
    if "pack" in parts:
        write_pack()
    if "quant" not in parts and "c1" not in parts:
        print("wrote", sorted(os.listdir(HERE)))
        return
    ref_moe, ref_quant, ref_lora = _import_reference()
    torch.manual_seed(0)
    out = {}
    # ---- quantize_int4 bytes + dequant values
    for name, (w, grp) in quant_cases().items():
        pk = ref_quant.quantize_int4(w, grp)
        out[f"quant.{name}.w"] = w.contiguous()
        out[f"quant.{name}.q"] = pk["q"]
        out[f"quant.{name}.scale"] = pk["scale"]
        out[f"quant.{name}.zero"] = pk["zero"]
        out[f"quant.{name}.deq_f32"] = ref_quant.dequant_int4_torch(pk["q"], pk["scale"], pk["zero"], torch.float32)
        out[f"quant.{name}.deq_bf16_torch"] = ref_quant.dequant_int4_torch(pk["q"], pk["scale"], pk["zero"],
                                                                           torch.bfloat16)
    save_file(out, os.path.join(HERE, "quant_int4.safetensors"))

    # ---- C1 end to end, fp32, through the reference's CPU path
    t = c1_inputs()
    out = {"in." + k: v.contiguous() for k, v in t.items()}
    gu4 = ref_quant.quantize_int4(t["gate_up"], 64)
    dn4 = ref_quant.quantize_int4(t["down"], 32)
    for k, v in gu4.items():
        out["bank.gate_up." + k] = v
    for k, v in dn4.items():
        out["bank.down." + k] = v
    bank = ref_moe.Int4Experts(gu4, dn4, dtype=torch.float32)
    sel = t["sel_ids"]
    gu_full = ref_quant.dequant_int4_torch(gu4["q"], gu4["scale"], gu4["zero"], torch.float32)
    dn_full = ref_quant.dequant_int4_torch(dn4["q"], dn4["scale"], dn4["zero"], torch.float32)
    # the selected experts keep their bf16-checkpoint values (pack.py:19-21): here the unquantized fp32 weights
    sel_gu, sel_dn = t["gate_up"][sel].clone(), t["down"][sel].clone()
    ex = ref_moe.LayerExperts(bank, sel.tolist(), sel_gu, sel_dn, group=32)
    H, I, Is, r = 64, 32, 32, 4
    exl = ref_lora.ExpertsLoRA(sel.tolist(), H, I, r, 8.0)
    shl = ref_lora.MLPLoRA(H, Is, r, 8.0)
    with torch.no_grad():
        for n in ("A_gate", "A_up", "A_down", "B_gate", "B_up", "B_down"):
            getattr(exl, n).copy_(t["ex_" + n])
            getattr(shl, n).copy_(t["sh_" + n])
    layer_lora = ref_lora.LayerLoRA(exl, shl)
    W = {"mlp.gate.weight": t["gate_w"],
         "mlp.shared_expert.gate_proj.weight": t["sh_gate"],
         "mlp.shared_expert.up_proj.weight": t["sh_up"],
         "mlp.shared_expert.down_proj.weight": t["sh_down"],
         "mlp.shared_expert_gate.weight": t["sh_gate_w"]}
    x = t["x"].clone().requires_grad_(True)
    captured = {}

    def stats(probs, topv, topi):
        captured["probs"], captured["topv"], captured["topi"] = probs.detach(), topv.detach(), topi.detach()

    y = ref_moe.moe_forward(x, W, ex, 2, layer_lora, stats=stats)
    y.backward(t["gy"])
    out["out.y"] = y.detach()
    out["out.dx"] = x.grad.detach()
    for k, v in captured.items():
        out["out." + k] = v
    for n in ("A_gate", "A_up", "A_down", "B_gate", "B_up", "B_down"):
        out["out.d_ex_" + n] = getattr(exl, n).grad.detach()
        out["out.d_sh_" + n] = getattr(shl, n).grad.detach()
    out["out.deq_gate_up"] = gu_full
    out["out.deq_down"] = dn_full
    # routed part alone, and the frozen-only layer (no selection), forward + dX
    with torch.no_grad():
        out["out.routed"] = ref_moe.routed_experts(t["x"], captured["topv"], captured["topi"], ex, exl)
    ex0 = ref_moe.LayerExperts(bank, group=32)
    x0 = t["x"].clone().requires_grad_(True)
    y0 = ref_moe.moe_forward(x0, W, ex0, 2)
    y0.backward(t["gy"])
    out["out.y_frozen_only"] = y0.detach()
    out["out.dx_frozen_only"] = x0.grad.detach()
    # Gemma-4 router on the same x (route_gemma4, smel/moe.py:170-180)
    g = torch.Generator().manual_seed(3)
    Wg = {"router.scale": 1 + 0.2 * torch.randn(H, generator=g),
          "router.proj.weight": torch.randn(8, H, generator=g) * 0.05,
          "router.per_expert_scale": 0.5 + torch.rand(8, generator=g)}
    pg, vg, ig = ref_moe.route_gemma4(t["x"], Wg, 2, 1e-6)
    for k, v in Wg.items():
        out["gemma." + k] = v
    out["gemma.probs"], out["gemma.topv"], out["gemma.topi"] = pg, vg, ig
    save_file(out, os.path.join(HERE, "c1_moe_fp32.safetensors"))
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main(set(sys.argv[1:]) or {"quant", "c1", "pack"})
