"""The packed-layer format (producer side) and exact LoRA merging: the API of the reference's smel/pack.py
(``pack_layer``, ``merge_experts``, ``merge_mlp``; same arguments, names, dtypes and results).

A packed layer is one flat dict of tensors (one ``layer_NN.safetensors`` on disk) that smel.stream.build_layer reads
back. It has three parts, in this order:
  * every tensor of the layer that is not a routed-expert weight, under its own name: floating tensors in the
    packing dtype (bf16), except the SSM parameters ``*A_log`` / ``*dt_bias`` and non-floating tensors, which keep
    their dtype (smel/pack.py:11-15);
  * with a selection: ``experts.sel.ids`` (int64 [k], on the host) and the selected experts' dense weights
    ``experts.sel.gate_up`` [k, 2I, H] / ``experts.sel.down`` [k, H, I] in the packing dtype (:16-21);
  * the whole routed bank in int4: ``experts.gate_up.{q,scale,zero}`` and ``experts.down.{q,scale,zero}`` (:22-24),
    each bank quantized by one launch of the HIP kernel smel_quantize_int4 (smel.quant.quantize_int4). Banks on the
    host are quantized on the current GPU and come back on the host.
"""
from __future__ import annotations

import torch

from .quant import quantize_int4

_EXPERTS = "mlp.experts."
_BANKS = (("gate_up", "mlp.experts.gate_up_proj"), ("down", "mlp.experts.down_proj"))
_KEEP_DTYPE_SUFFIXES = ("A_log", "dt_bias")


def _stored_dtype(name: str, v: torch.Tensor, dtype):
    if not v.is_floating_point() or name.endswith(_KEEP_DTYPE_SUFFIXES):
        return v.dtype
    return dtype


def _dense_part(t: dict, dtype) -> dict:
    """Every non-expert tensor under its own name, in its stored dtype, contiguous."""
    return {k: v.to(_stored_dtype(k, v, dtype)).contiguous() for k, v in t.items() if not k.startswith(_EXPERTS)}


def _selected_part(t: dict, sel_ids, dtype) -> dict:
    """The selected experts' dense weights, gathered from the fused bf16 tensors (nothing for no selection)."""
    if sel_ids is None or len(sel_ids) == 0:
        return {}
    ids = torch.as_tensor([int(e) for e in sel_ids], dtype=torch.int64)
    part = {"experts.sel.ids": ids}
    for name, key in _BANKS:
        w = t[key]
        part[f"experts.sel.{name}"] = w[ids.to(w.device)].to(dtype).contiguous()
    return part


def _bank_part(t: dict, group: int) -> dict:
    """Both banks in int4 (q, scale, zero), group-wise along each bank's input dim."""
    part = {}
    for name, key in _BANKS:
        for field, v in quantize_int4(t[key], group).items():
            part[f"experts.{name}.{field}"] = v
    return part


def pack_layer(t: dict, sel_ids=None, group: int = 64, dtype=torch.bfloat16) -> dict:
    """t: the tensors of one layer under their checkpoint names relative to the layer (the routed experts fused as
    ``mlp.experts.gate_up_proj`` [E, 2I, H] and ``mlp.experts.down_proj`` [E, H, I]) -> the packed layer
    (smel/pack.py:8-25). A missing expert tensor raises KeyError; an input dim that is not a multiple of ``group``
    raises AssertionError."""
    out = _dense_part(t, dtype)
    for key in (k for _, k in _BANKS):
        if key not in t:
            raise KeyError(key)
        K = t[key].shape[-1]
        assert K % group == 0 and group % 2 == 0, f"{key}: input dim {K} is not a multiple of the (even) group {group}"
    out.update(_selected_part(t, sel_ids, dtype))
    out.update(_bank_part(t, group))
    return out


def _add_delta_(w: torch.Tensor, d: torch.Tensor) -> None:
    """w <- dtype(fp32(w) + d): the sum in fp32, one rounding to w's dtype."""
    w.copy_(w.float() + d.to(w.device))


@torch.no_grad()
def merge_experts(gate_up: torch.Tensor, down: torch.Tensor, lora) -> tuple:
    """Copies of the fused expert weights with each selected expert's LoRA delta (scale B) A added in fp32
    (smel/pack.py:28-38). ``lora``: an ExpertsLoRA (slot j adapts expert ``expert_ids[j]``; slots apply in order)."""
    gu, dn = gate_up.clone(), down.clone()
    inter = dn.shape[2]
    for j, e in enumerate(lora.expert_ids.tolist()):
        d_gate, d_up, d_down = lora.delta(j)
        _add_delta_(gu[e, :inter], d_gate)
        _add_delta_(gu[e, inter:], d_up)
        _add_delta_(dn[e], d_down)
    return gu, dn


@torch.no_grad()
def merge_mlp(gate_w, up_w, down_w, lora) -> tuple:
    """(gate, up, down) weights of a gated MLP with its MLPLoRA delta added in fp32, each rounded once to its own
    dtype (smel/pack.py:41-45)."""
    return tuple((w.float() + d.to(w.device)).to(w.dtype) for w, d in zip((gate_w, up_w, down_w), lora.delta()))
