"""Shared test helpers: build the oracle layer from the C1 golden fixture, tolerance checks."""
import torch

from oracle import moe_ref as R

QUANT_CASES = ("normal", "outlier", "g32", "grid", "e20")
LORA_NAMES = ("A_gate", "A_up", "A_down", "B_gate", "B_up", "B_down")


def c1_layer(t, with_sel=True, deq_dtype=torch.float32) -> R.OracleLayer:
    """The C1 layer exactly as tests/golden/make_golden.py handed it to the reference."""
    frozen = {"gate_up": {k: t["bank.gate_up." + k] for k in ("q", "scale", "zero")},
              "down": {k: t["bank.down." + k] for k in ("q", "scale", "zero")}}
    L = R.OracleLayer(gate_w=t["in.gate_w"], frozen=frozen, int4=True, deq_dtype=deq_dtype, expert_group=32)
    L.shared = {"gate_up": torch.cat((t["in.sh_gate"], t["in.sh_up"])), "down": t["in.sh_down"],
                "gate_w": t["in.sh_gate_w"]}
    if with_sel:
        sel = t["in.sel_ids"]
        L.sel_ids = sel.tolist()
        L.sel_gate_up, L.sel_down = t["in.gate_up"][sel].clone(), t["in.down"][sel].clone()
        L.ex_lora = {n: t["in.ex_" + n] for n in LORA_NAMES}
        L.ex_scale = 2.0
        L.sh_lora = {n: t["in.sh_" + n] for n in LORA_NAMES}
        L.sh_scale = 2.0
    return L


def assert_close_bf16(out, ref, name="", rel=2e-2, cos=0.9999):
    """The bf16 bar: ||out-ref||/||ref|| <= rel, max|out-ref| <= rel * max|ref| and cosine >= cos."""
    e = R.rel_err(out, ref)
    c = R.cosine(out, ref)
    m = ((out.double() - ref.double()).abs().max() / ref.double().abs().max().clamp_min(1e-30)).item()
    assert e <= rel and m <= rel and c >= cos, f"{name}: rel {e:.3e} max {m:.3e} cos {c:.6f}"
    return e, m, c


def to_device_layer(ol: R.OracleLayer, device, dtype=torch.bfloat16):
    """The oracle's layer as the drop-in API's objects on ``device``: (W dict, LayerExperts, LayerLoRA or None), the
    floating weights in ``dtype`` (bf16, or fp32 for the fp32 path, whose int4 bank then keeps the oracle's
    dequant dtype as Int4Experts.dtype)."""
    from smel.lora import ExpertsLoRA, LayerLoRA, MLPLoRA
    from smel.moe import BF16Experts, Int4Experts, LayerExperts

    bf = lambda t: t.to(device=device, dtype=dtype).contiguous()
    W = {"mlp.gate.weight": bf(ol.gate_w)}
    if ol.shared is not None:
        Is = ol.shared["down"].shape[1]
        W["mlp.shared_expert.gate_proj.weight"] = bf(ol.shared["gate_up"][:Is])
        W["mlp.shared_expert.up_proj.weight"] = bf(ol.shared["gate_up"][Is:])
        W["mlp.shared_expert.down_proj.weight"] = bf(ol.shared["down"])
        W["mlp.shared_expert_gate.weight"] = bf(ol.shared["gate_w"])
    if ol.int4:
        dev = lambda d: {k: v.to(device).contiguous() for k, v in d.items()}
        bank = Int4Experts(dev(ol.frozen["gate_up"]), dev(ol.frozen["down"]),
                           dtype=ol.deq_dtype if dtype == torch.float32 else torch.bfloat16)
    else:
        bank = BF16Experts(bf(ol.frozen["gate_up"]), bf(ol.frozen["down"]))
    if ol.sel_ids:
        ex = LayerExperts(bank, ol.sel_ids, bf(ol.sel_gate_up), bf(ol.sel_down), group=32, act=ol.act)
    else:
        ex = LayerExperts(bank, group=32, act=ol.act)
    lora = None
    if ol.ex_lora is not None or ol.sh_lora is not None:
        exl = shl = None
        if ol.ex_lora is not None:
            r, H = ol.ex_lora["A_gate"].shape[1:]
            I = ol.ex_lora["A_down"].shape[2]
            exl = ExpertsLoRA(ol.sel_ids, H, I, r, ol.ex_scale * r)
            with torch.no_grad():
                for n in LORA_NAMES:
                    getattr(exl, n).copy_(ol.ex_lora[n])
            exl = exl.to(device)
        if ol.sh_lora is not None:
            r, H = ol.sh_lora["A_gate"].shape
            Is = ol.sh_lora["A_down"].shape[1]
            shl = MLPLoRA(H, Is, r, ol.sh_scale * r)
            with torch.no_grad():
                for n in LORA_NAMES:
                    getattr(shl, n).copy_(ol.sh_lora[n])
            shl = shl.to(device)
        lora = LayerLoRA(exl, shl)
    return W, ex, lora
