"""LoRA parameter containers of the selected experts and the shared MLP (the types of smel/lora.py:14-58, 86-90).

Parameters are fp32 nn.Parameters with the reference's shapes and init (A: kaiming_uniform(a=sqrt(5)) per [r, in]
matrix, B: zeros); slot j of ExpertsLoRA belongs to expert ``expert_ids[j]``. The LoRA products themselves run inside
the MoE kernels (a 32-wide K-extension of the expert GEMMs), see ``smel.moe``.
"""
from __future__ import annotations

import math

import torch
from torch import nn


def _init_a(t: torch.Tensor):
    for m in t.reshape(-1, *t.shape[-2:]):
        nn.init.kaiming_uniform_(m, a=math.sqrt(5))


class ExpertsLoRA(nn.Module):
    """LoRA of k selected experts: A_gate/A_up [k, r, H], B_gate/B_up [k, I, r], A_down [k, r, I], B_down [k, H, r]."""

    def __init__(self, expert_ids, hidden: int, inter: int, r: int = 16, alpha: float = 32.0):
        super().__init__()
        k = len(expert_ids)
        self.register_buffer("expert_ids", torch.as_tensor(list(expert_ids), dtype=torch.long), persistent=True)
        self.r, self.alpha, self.scale = r, alpha, alpha / r
        self.A_gate = nn.Parameter(torch.empty(k, r, hidden))
        self.B_gate = nn.Parameter(torch.zeros(k, inter, r))
        self.A_up = nn.Parameter(torch.empty(k, r, hidden))
        self.B_up = nn.Parameter(torch.zeros(k, inter, r))
        self.A_down = nn.Parameter(torch.empty(k, r, inter))
        self.B_down = nn.Parameter(torch.zeros(k, hidden, r))
        for a in (self.A_gate, self.A_up, self.A_down):
            _init_a(a.data)

    def delta(self, j: int):
        s = self.scale
        return (s * self.B_gate[j].float() @ self.A_gate[j].float(),
                s * self.B_up[j].float() @ self.A_up[j].float(),
                s * self.B_down[j].float() @ self.A_down[j].float())


class MLPLoRA(nn.Module):
    """LoRA of a plain gated MLP (the shared expert / Gemma's dense MLP): A_* [r, in], B_* [out, r]."""

    def __init__(self, hidden: int, inter: int, r: int = 16, alpha: float = 32.0):
        super().__init__()
        self.r, self.alpha, self.scale = r, alpha, alpha / r
        self.A_gate = nn.Parameter(torch.empty(r, hidden))
        self.B_gate = nn.Parameter(torch.zeros(inter, r))
        self.A_up = nn.Parameter(torch.empty(r, hidden))
        self.B_up = nn.Parameter(torch.zeros(inter, r))
        self.A_down = nn.Parameter(torch.empty(r, inter))
        self.B_down = nn.Parameter(torch.zeros(hidden, r))
        for a in (self.A_gate, self.A_up, self.A_down):
            _init_a(a.data)

    def delta(self):
        s = self.scale
        return (s * self.B_gate.float() @ self.A_gate.float(),
                s * self.B_up.float() @ self.A_up.float(),
                s * self.B_down.float() @ self.A_down.float())


def lora_linear(x, w, A, B, scale):
    """x w^T + scale (x A^T) B^T with the LoRA factors cast to x's dtype (smel/lora.py:61-69). A dense helper of the
    API; the MoE layer itself runs its LoRA products inside the grouped-GEMM kernels."""
    y = x @ w.t()
    if A is None:
        return y
    if x.dim() == 2:
        return torch.addmm(y, x @ A.to(x.dtype).t(), B.to(x.dtype).t(), alpha=scale)
    return y + scale * ((x @ A.to(x.dtype).t()) @ B.to(x.dtype).t())


def lora_gate_up(x, w_gate_up, A_gate, B_gate, A_up, B_up, scale):
    """(gate, up) of a gated MLP from one stacked [2I, H] weight (smel/lora.py:72-83); dense helper of the API."""
    I = w_gate_up.shape[0] // 2
    base = x @ w_gate_up.t()
    if A_gate is None:
        return base[:, :I], base[:, I:]
    r = A_gate.shape[0]
    xa = x @ torch.cat((A_gate, A_up)).to(x.dtype).t()
    g = torch.addmm(base[:, :I], xa[:, :r], B_gate.to(x.dtype).t(), alpha=scale)
    u = torch.addmm(base[:, I:], xa[:, r:], B_up.to(x.dtype).t(), alpha=scale)
    return g, u


class LayerLoRA(nn.Module):
    def __init__(self, experts: ExpertsLoRA | None, shared: MLPLoRA | None):
        super().__init__()
        self.experts = experts
        self.shared = shared


class BlockLoRA(nn.Module):
    """All LoRA modules of a block of layers, keyed by absolute layer index (smel/lora.py:93-125)."""

    def __init__(self, layers: dict):
        super().__init__()
        self.layers = nn.ModuleDict({str(k): v for k, v in layers.items()})

    def get(self, l: int):
        return self.layers[str(l)] if str(l) in self.layers else None

    @classmethod
    def build(cls, selection: dict, hidden: int, inter: int, shared_inter: int, r: int, alpha: float,
              shared: bool = True):
        layers = {}
        for l, ids in selection.items():
            ex = ExpertsLoRA(ids, hidden, inter, r, alpha) if len(ids) else None
            sh = MLPLoRA(hidden, shared_inter, r, alpha) if shared else None
            layers[int(l)] = LayerLoRA(ex, sh)
        return cls(layers)
