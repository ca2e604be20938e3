"""LoRA parameter sets of the selected routed experts and of the shared / dense MLP: the adapter format of the
reference's smel/lora.py (classes ExpertsLoRA, MLPLoRA, LayerLoRA, BlockLoRA; parameters A_gate, B_gate, A_up,
B_up, A_down, B_down in that order, fp32, A [.., r, in] uniform in +-1/sqrt(in) (kaiming_uniform with a = sqrt(5)),
B [.., out, r] zero), so adapters written by either load into the other.

The MoE layer never multiplies these factors in Python: smel.moe lays them out as a 32-wide K-extension of the
grouped-GEMM kernels. ``lora_linear`` / ``lora_gate_up`` are the dense helpers of the API (torch ops).
"""
from __future__ import annotations

import json
import math
import os

import torch
import torch.nn.functional as F
from torch import nn

_PROJ = ("gate", "up", "down")


def _uniform_fan_in(a: torch.Tensor) -> torch.Tensor:
    """Every [r, in] matrix of ``a`` uniform in +-1/sqrt(in): kaiming_uniform_ with a = sqrt(5) gives
    gain sqrt(2 / (1 + 5)) and bound gain * sqrt(3 / in), which is that."""
    bound = 1.0 / math.sqrt(a.shape[-1])
    with torch.no_grad():
        for m in a.view(-1, *a.shape[-2:]):
            m.uniform_(-bound, bound)
    return a


class _LoRASet(nn.Module):
    """The six factors of a gated MLP's LoRA, with ``lead`` leading dims (() for one MLP, (k,) for k experts):
    A_p [*lead, r, in_p], B_p [*lead, out_p, r] for p = gate, up (in = hidden, out = inter) and down (in = inter,
    out = hidden); scale = alpha / r."""

    def __init__(self, lead: tuple, hidden: int, inter: int, r: int, alpha: float):
        super().__init__()
        self.r, self.alpha, self.scale = r, alpha, alpha / r
        io = {"gate": (hidden, inter), "up": (hidden, inter), "down": (inter, hidden)}
        for p in _PROJ:
            fan_in, fan_out = io[p]
            setattr(self, f"A_{p}", nn.Parameter(_uniform_fan_in(torch.empty(*lead, r, fan_in))))
            setattr(self, f"B_{p}", nn.Parameter(torch.zeros(*lead, fan_out, r)))

    def _deltas(self, idx):
        """(scale B_p) A_p for the three projections at index ``idx`` of the leading dims (fp32; B is scaled before
        the product, the order of smel/lora.py:31-36, so merged weights round as the reference's)."""
        def one(p):
            return torch.matmul(getattr(self, f"B_{p}")[idx].float() * self.scale, getattr(self, f"A_{p}")[idx].float())
        return tuple(one(p) for p in _PROJ)


class ExpertsLoRA(_LoRASet):
    """LoRA of k selected experts of one layer (smel/lora.py:14-36): slot j belongs to expert ``expert_ids[j]``."""

    def __init__(self, expert_ids, hidden: int, inter: int, r: int = 16, alpha: float = 32.0):
        ids = [int(e) for e in expert_ids]
        super().__init__((len(ids),), hidden, inter, r, alpha)
        self.register_buffer("expert_ids", torch.tensor(ids, dtype=torch.long), persistent=True)

    def delta(self, j: int):
        """Dense weight deltas of slot j: (d_gate [I, H], d_up [I, H], d_down [H, I]), fp32."""
        return self._deltas(j)


class MLPLoRA(_LoRASet):
    """LoRA of one gated MLP: the shared expert, or Gemma 4's dense MLP (smel/lora.py:39-58)."""

    def __init__(self, hidden: int, inter: int, r: int = 16, alpha: float = 32.0):
        super().__init__((), hidden, inter, r, alpha)

    def delta(self):
        return self._deltas(())


def _add_low_rank(y, xa, B, scale):
    """y + scale (xa B^T), B cast to the rows' dtype. For rows given as a matrix, one addmm: the low-rank product's
    sum, its scaling and the add round once (the reference's epilogue form); other shapes scale and add the rounded
    product, as the reference does for them."""
    bt = B.to(xa.dtype).t()
    if xa.dim() == 2:
        return torch.addmm(y, xa, bt, alpha=scale)
    return y + scale * (xa @ bt)


def lora_linear(x, w, A, B, scale):
    """x w^T + scale (x A^T) B^T with the LoRA factors in x's dtype (smel/lora.py:61-69)."""
    y = x @ w.t()
    if A is None:
        return y
    return _add_low_rank(y, x @ A.to(x.dtype).t(), B, scale)


def lora_gate_up(x, w_gate_up, A_gate, B_gate, A_up, B_up, scale):
    """(gate, up) of a gated MLP from its stacked [2I, H] weight (smel/lora.py:72-83): one base GEMM over the stacked
    weight and one rank-2r projection x [A_gate; A_up]^T, whose two halves go through B_gate and B_up into the gate
    and up halves. Rows of any leading shape (flattened to a matrix for the products)."""
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    I = w_gate_up.shape[0] // 2
    base = x2 @ w_gate_up.t()
    g, u = base[:, :I], base[:, I:]
    if A_gate is not None:
        r = A_gate.shape[0]
        xa = x2 @ torch.cat((A_gate, A_up)).to(x.dtype).t()
        g, u = _add_low_rank(g, xa[:, :r], B_gate, scale), _add_low_rank(u, xa[:, r:], B_up, scale)
    return g.reshape(*lead, I), u.reshape(*lead, I)


class LayerLoRA(nn.Module):
    """The LoRA of one layer: ``experts`` (ExpertsLoRA or None) and ``shared`` (MLPLoRA or None)."""

    def __init__(self, experts: ExpertsLoRA | None, shared: MLPLoRA | None):
        super().__init__()
        self.experts = experts
        self.shared = shared


class BlockLoRA(nn.Module):
    """The LoRA of a block of layers, keyed by absolute layer index (smel/lora.py:93-125)."""

    def __init__(self, layers: dict):
        super().__init__()
        self.layers = nn.ModuleDict({str(k): v for k, v in layers.items()})

    def get(self, l: int):
        key = str(l)
        return self.layers[key] if key in self.layers else None

    @classmethod
    def build(cls, selection: dict, hidden: int, inter: int, shared_inter: int, r: int, alpha: float,
              shared: bool = True):
        """selection {layer: [expert ids]} -> one LayerLoRA per layer (no ExpertsLoRA for an empty selection)."""
        def layer(ids):
            ex = ExpertsLoRA(ids, hidden, inter, r, alpha) if len(ids) else None
            return LayerLoRA(ex, MLPLoRA(hidden, shared_inter, r, alpha) if shared else None)
        return cls({int(l): layer(ids) for l, ids in selection.items()})

    @classmethod
    def load(cls, path, dims, device="cuda"):
        """An adapter folder (adapter_config.json + adapter.safetensors, the reference trainer's output format) ->
        (BlockLoRA on ``device``, the config dict). ``dims`` supplies hidden, moe_inter and shared_inter."""
        from safetensors.torch import load_file
        with open(os.path.join(path, "adapter_config.json")) as f:
            meta = json.load(f)
        sel = {int(l): ids for l, ids in meta["experts"].items()}
        block = cls.build(sel, dims.hidden, dims.moe_inter, dims.shared_inter, meta["r"], meta["alpha"],
                          shared=meta["shared_lora"])
        block.load_state_dict(load_file(os.path.join(path, "adapter.safetensors")))
        return block.to(device), meta
