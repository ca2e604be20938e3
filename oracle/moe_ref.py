"""CPU restatement (torch, fp32 or fp64) of SMEL FT's MoE-layer hot path — TEST INFRASTRUCTURE ONLY.

The checker for the HIP kernels and the timed CPU baseline of bench.py. Nothing in the product path imports it.
Every function cites the reference code it restates (paths relative to the reference repository root).

Numerics follow the reference's own CPU path: stable-argsort dispatch, int4 dequant per group of experts, per-expert
matmul loops, fp32 weighted combine, and torch autograd for everything except the frozen experts, whose backward
re-dequantizes the weights (smel/moe.py:120-143). Pass ``dtype=torch.float64`` for a higher-precision reference.

PINNED — what checks each function against something other than its own formula (tests that do it in brackets):
  quantize_int4 ......... golden bytes written by the reference itself [test_oracle.py::test_quantize_golden]
  dequant_int4 .......... golden fp32 values of the reference + closed form RNE(q*s+z) through the C restatement
                          [test_oracle.py::test_dequant_golden, ::test_dequant_c_matches]
  dequant_int4_bf16math . golden bf16 values of the reference's torch fallback [::test_dequant_golden]
  topk_lowest_index ..... torch.topk on tie-free rows + brute-force sort on tied rows [::test_topk_*]
  route ................. golden probs/topv/topi of the reference (C1) [::test_route_golden]
  route_gemma4 .......... golden values of the reference (C1 input) [::test_route_gemma4_golden]
  dispatch .............. numpy stable argsort + the C counting sort + invariants [::test_dispatch_*]
  act / act_and_grad .... torch.autograd.gradcheck in fp64 + torch.nn.functional [::test_act_grad]
  lora_linear/_gate_up .. plain fp64 formula and its autograd [::test_lora_plain_formula]
  routed_experts ........ golden reference output (C1) [::test_routed_golden]
  gemma4_moe_block ...... composed of the pinned parts (route_gemma4, mlp_lora, routed_experts) and the pinned torch
                          RMSNorm of norm_ref; fp64 per-token brute force of the whole block [::test_gemma4_block]
  moe_forward + backward  golden reference y, dX, LoRA dA/dB (C1, with and without selected experts), fp64
                          brute force per token [::test_moe_golden, ::test_moe_bruteforce]
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch
import torch.nn.functional as F

# --------------------------------------------------------------------------------------------- int4 format (A7/A8)


def _q4_candidate(wg, lo, hi):
    """One clip candidate (smel/quant.py:5-11): scale/zero are rounded to bf16 before q is computed."""
    scale = ((hi - lo) / 15).clamp_min(1e-8).to(torch.bfloat16).float()
    zero = lo.to(torch.bfloat16).float()
    q = torch.round((wg - zero) / scale).clamp_(0, 15)
    return q, scale, zero


def quantize_int4(w: torch.Tensor, group: int = 64, clip_search=(1.0, 0.95, 0.9, 0.85, 0.8)) -> dict:
    """Group-wise asymmetric int4 (smel/quant.py:14-44). Returns {"q": uint8 [..., K/2] (low nibble = even k),
    "scale": bf16 [..., K/group], "zero": bf16 [..., K/group]}. For each group the [min, max] range is shrunk about
    its midpoint by each clip factor; a later candidate replaces the kept one only if its squared error is strictly
    smaller. 3-D inputs with more than 16 experts are processed 16 experts at a time (smel/quant.py:18-20), which
    keeps the fp32 reduction shapes identical to the reference."""
    if w.dim() == 3 and w.shape[0] > 16:
        parts = [quantize_int4(w[i:i + 16], group, clip_search) for i in range(0, w.shape[0], 16)]
        return {k: torch.cat([p[k] for p in parts]) for k in parts[0]}
    K = w.shape[-1]
    if K % group or group % 2:
        raise AssertionError(f"K={K} must be a multiple of the (even) group {group}")
    wg = w.float().reshape(*w.shape[:-1], K // group, group)
    lo0, hi0 = wg.amin(-1, keepdim=True), wg.amax(-1, keepdim=True)
    mid = (lo0 + hi0) / 2
    best_err = best_q = best_s = best_z = None
    for c in clip_search or (1.0,):
        q, s, z = _q4_candidate(wg, mid + (lo0 - mid) * c, mid + (hi0 - mid) * c)
        err = (q * s + z - wg).pow(2).sum(-1, keepdim=True)
        if best_err is None:
            best_err, best_q, best_s, best_z = err, q, s, z
            continue
        take = err < best_err
        best_err = torch.where(take, err, best_err)
        best_q = torch.where(take, q, best_q)
        best_s = torch.where(take, s, best_s)
        best_z = torch.where(take, z, best_z)
    q = best_q.to(torch.uint8).reshape(*w.shape[:-1], K)
    return {"q": (q[..., 0::2] | (q[..., 1::2] << 4)).contiguous(),
            "scale": best_s.squeeze(-1).to(torch.bfloat16),
            "zero": best_z.squeeze(-1).to(torch.bfloat16)}


def unpack_nibbles(q: torch.Tensor) -> torch.Tensor:
    """uint8 [..., K/2] -> uint8 [..., K]; k even = low nibble, k odd = high nibble (smel/quant.py:42, 59-66)."""
    return torch.stack((q & 0xF, q >> 4), dim=-1).reshape(*q.shape[:-1], q.shape[-1] * 2)


def dequant_int4(q, scale, zero, dtype=torch.bfloat16) -> torch.Tensor:
    """GPU-kernel semantics of the reference (Triton ``_dq4_kernel``, smel/quant.py:51-67): w = q*s + z evaluated in
    fp32 (q*s is exact: q <= 15 and s is bf16), then one round-to-nearest-even to ``dtype``."""
    K = q.shape[-1] * 2
    G = scale.shape[-1]
    qf = unpack_nibbles(q).float().reshape(*q.shape[:-1], G, K // G)
    w = qf * scale.float().unsqueeze(-1) + zero.float().unsqueeze(-1)
    return w.reshape(*q.shape[:-1], K).to(dtype)


def dequant_int4_bf16math(q, scale, zero, dtype=torch.bfloat16) -> torch.Tensor:
    """CPU-fallback semantics of the reference (``dequant_int4_torch``, smel/quant.py:87-94): the product and the
    add are each rounded to ``dtype`` (two roundings in bf16)."""
    K = q.shape[-1] * 2
    G = scale.shape[-1]
    w = unpack_nibbles(q).reshape(*q.shape[:-1], G, K // G).to(dtype)
    w = w * scale.unsqueeze(-1).to(dtype) + zero.unsqueeze(-1).to(dtype)
    return w.reshape(*q.shape[:-1], K)


def rel_err(a, b) -> float:
    """||a - b|| / ||b|| in fp64 (the reference's smel/quant.py:108-110 measure)."""
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def cosine(a, b) -> float:
    a, b = a.double().flatten(), b.double().flatten()
    return (a @ b / (a.norm() * b.norm()).clamp_min(1e-300)).item()


# ------------------------------------------------------------------------------------------------- router (A1/A2)


def topk_lowest_index(p: torch.Tensor, k: int):
    """Top-k along the last dim, sorted by value descending; among equal values the lower index comes first. This
    is the deterministic rule the kernels implement; torch.topk gives the same result whenever the row has no tie
    within its top k+1 (its own order among ties is unspecified, and differs between CPU and GPU builds)."""
    # a stable sort of -value keeps equal values in index order: lexicographic (-value, index)
    order = torch.sort(-p, dim=-1, stable=True).indices
    topi = order[..., :k]
    return p.gather(-1, topi), topi


def route(x2d, gate_w, top_k, logits=None):
    """smel/moe.py:162-167: logits = x W^T (in x's dtype), probs = softmax in fp32, top-k, renormalised, topv cast
    back to the logits dtype. ``logits`` may be given to route identical logits (bit-exact id checks)."""
    if logits is None:
        logits = F.linear(x2d, gate_w)
    # fp32 as in the reference; an fp64 oracle run keeps fp64
    probs = torch.softmax(logits, dim=-1, dtype=torch.promote_types(torch.float32, logits.dtype))
    topv, topi = topk_lowest_index(probs, top_k)
    topv = topv / topv.sum(dim=-1, keepdim=True)
    return probs, topv.to(logits.dtype), topi


def route_gemma4(h, W, top_k, eps, forced_topi=None):
    """smel/moe.py:170-180: weightless RMSNorm of the residual stream in fp32, x router.scale x H^-0.5, logits,
    softmax fp32, top-k, renormalise, x per_expert_scale of the chosen experts. ``forced_topi`` replaces the chosen
    ids (topv stays differentiable through the softmax), as :func:`moe_forward` forces routing."""
    hf = h.float()
    x = (hf * torch.pow(hf.pow(2).mean(-1, keepdim=True) + eps, -0.5)).type_as(h)
    x = x * W["router.scale"] * h.shape[-1] ** -0.5
    logits = F.linear(x, W["router.proj.weight"])
    probs = torch.softmax(logits, dim=-1, dtype=torch.float32)
    if forced_topi is None:
        topv, topi = topk_lowest_index(probs, top_k)
    else:
        topi = forced_topi.long()
        topv = probs.gather(1, topi)
    topv = topv / topv.sum(dim=-1, keepdim=True)
    return probs, topv * W["router.per_expert_scale"][topi], topi


# --------------------------------------------------------------------------------------------------- dispatch (A3)


def dispatch(topi: torch.Tensor, n_experts: int):
    """smel/moe.py:216-223 plus the inverse of smel/moe.py:249-250, as a stable counting sort.
    Returns (order, tok, counts, offsets, inv), all int64:
      order[j]  = flat slot p = t*K + k stored at sorted position j (experts ascending, p ascending within one);
      tok[j]    = order[j] // K;  counts[e] = #slots routed to e;  offsets = exclusive cumsum (length E+1);
      inv[p]    = sorted position of slot p."""
    flat = topi.reshape(-1).long()
    K = topi.shape[-1]
    counts = torch.bincount(flat, minlength=n_experts)
    offsets = torch.zeros(n_experts + 1, dtype=torch.long)
    offsets[1:] = torch.cumsum(counts, 0)
    cursor = offsets[:-1].clone()
    order = torch.empty_like(flat)
    for p, e in enumerate(flat.tolist()):   # the textbook stable counting sort (small inputs)
        order[cursor[e]] = p
        cursor[e] += 1
    inv = torch.empty_like(order)
    inv[order] = torch.arange(order.numel())
    return order, order // K, counts, offsets, inv


def dispatch_fast(topi: torch.Tensor, n_experts: int):
    """Same result as :func:`dispatch` through torch's stable argsort (used at large sizes)."""
    flat = topi.reshape(-1).long()
    order = torch.argsort(flat, stable=True)
    counts = torch.bincount(flat, minlength=n_experts)
    offsets = torch.zeros(n_experts + 1, dtype=torch.long)
    offsets[1:] = torch.cumsum(counts, 0)
    inv = torch.empty_like(order)
    inv[order] = torch.arange(order.numel())
    return order, order // topi.shape[-1], counts, offsets, inv


# ----------------------------------------------------------------------------------------------- activations (A9)

GELU_C = math.sqrt(2.0 / math.pi)


def act(x, name):
    """smel/moe.py:91-96."""
    if name == "silu":
        return F.silu(x)
    if name == "gelu_tanh":
        return F.gelu(x, approximate="tanh")
    raise ValueError(f"unknown activation {name}")


def act_and_grad(g, name):
    """smel/moe.py:99-107: (act(g), act'(g)) in g's dtype."""
    if name == "silu":
        s = torch.sigmoid(g)
        return g * s, s * (1 + g * (1 - s))
    if name == "gelu_tanh":
        t = torch.tanh(GELU_C * (g + 0.044715 * g ** 3))
        return 0.5 * g * (1 + t), 0.5 * (1 + t) + 0.5 * g * (1 - t * t) * GELU_C * (1 + 3 * 0.044715 * g * g)
    raise ValueError(f"unknown activation {name}")


# ------------------------------------------------------------------------------------------------ LoRA (A11/A12)


def lora_linear(x, w, A, B, scale):
    """smel/lora.py:61-69: x w^T + scale (x A^T) B^T, LoRA factors cast to x's dtype."""
    y = x @ w.t()
    if A is None:
        return y
    return y + scale * ((x @ A.to(x.dtype).t()) @ B.to(x.dtype).t())


def lora_gate_up(x, w_gate_up, A_gate, B_gate, A_up, B_up, scale):
    """smel/lora.py:72-83: gate and up of a gated MLP from one stacked [2I, H] weight."""
    I = w_gate_up.shape[0] // 2
    base = x @ w_gate_up.t()
    if A_gate is None:
        return base[:, :I], base[:, I:]
    r = A_gate.shape[0]
    xa = x @ torch.cat((A_gate, A_up)).to(x.dtype).t()
    g = base[:, :I] + scale * (xa[:, :r] @ B_gate.to(x.dtype).t())
    u = base[:, I:] + scale * (xa[:, r:] @ B_up.to(x.dtype).t())
    return g, u


def mlp_lora(x, w_gate_up, w_down, lora: dict | None, scale: float, act_name="silu"):
    """smel/moe.py:183-194 with the stacked gate/up weight: down(act(gate(x)) * up(x)), LoRA on all three."""
    L = lora or {}
    g, u = lora_gate_up(x, w_gate_up, L.get("A_gate"), L.get("B_gate"), L.get("A_up"), L.get("B_up"), scale)
    return lora_linear(act(g, act_name) * u, w_down, L.get("A_down"), L.get("B_down"), scale)


# ------------------------------------------------------------------------------------------- layer description


@dataclass
class OracleLayer:
    """Everything one MoE layer holds (the W dict of smel/moe.py:255-263 plus LayerExperts and LayerLoRA), as CPU
    tensors. ``frozen`` is either {"gate_up": {q,scale,zero}, "down": {q,scale,zero}} (int4 bank) or
    {"gate_up": [E,2I,H], "down": [E,H,I]} (bf16 bank). LoRA dicts hold A_gate, B_gate, A_up, B_up, A_down, B_down
    (fp32, [k, ...] for experts)."""
    gate_w: torch.Tensor
    frozen: dict
    int4: bool = True
    sel_ids: list = field(default_factory=list)
    sel_gate_up: torch.Tensor | None = None
    sel_down: torch.Tensor | None = None
    ex_lora: dict | None = None
    ex_scale: float = 0.0
    shared: dict | None = None          # {"gate_up": [2Is,H], "down": [H,Is], "gate_w": [1,H]} or None
    sh_lora: dict | None = None
    sh_scale: float = 0.0
    act: str = "silu"
    expert_group: int = 32               # experts dequantized at once (configs/default.yaml:47)
    deq_dtype: torch.dtype = torch.bfloat16   # dtype the int4 bank is dequantized to (Int4Experts.dtype)

    @property
    def E(self):
        return self.gate_w.shape[0]

    @classmethod
    def from_api(cls, W: dict, ex, lora=None, router_key: str = "mlp.gate.weight"):
        """The layer held by the drop-in API's objects (the W dict of smel/moe.py:255-263, a LayerExperts and a
        LayerLoRA; device tensors are copied to the CPU): the oracle then computes on exactly the weights a GPU layer
        was built with. The LoRA of ``lora.shared`` is kept in ``sh_lora`` also without a shared expert (Gemma 4's
        dense MLP takes the layer's shared LoRA, smel/layer_runner.py:249-254)."""
        c = lambda t: t.detach().cpu()
        fz = ex.frozen
        int4 = hasattr(fz, "gu")
        frozen = ({"gate_up": {k: c(v) for k, v in fz.gu.items()}, "down": {k: c(v) for k, v in fz.dn.items()}}
                  if int4 else {"gate_up": c(fz.gate_up), "down": c(fz.down)})
        sel = [int(e) for e in ex.sel_ids] if ex.sel_ids is not None else []
        L = cls(gate_w=c(W[router_key]), frozen=frozen, int4=int4, sel_ids=sel, act=ex.act,
                deq_dtype=getattr(fz, "dtype", torch.bfloat16))
        names = ("A_gate", "B_gate", "A_up", "B_up", "A_down", "B_down")
        if sel:
            L.sel_gate_up, L.sel_down = c(ex.sel_gate_up), c(ex.sel_down)
            if lora is not None and lora.experts is not None:
                L.ex_lora = {n: c(getattr(lora.experts, n)).float() for n in names}
                L.ex_scale = float(lora.experts.scale)
        pre = "mlp.shared_expert."
        if pre + "down_proj.weight" in W:
            gu = W.get(pre + "gate_up_proj.weight")
            if gu is None:
                gu = torch.cat((W[pre + "gate_proj.weight"], W[pre + "up_proj.weight"]))
            L.shared = {"gate_up": c(gu), "down": c(W[pre + "down_proj.weight"]),
                        "gate_w": c(W["mlp.shared_expert_gate.weight"]).reshape(1, -1)}
        if lora is not None and lora.shared is not None:
            L.sh_lora = {n: c(getattr(lora.shared, n)).float() for n in names}
            L.sh_scale = float(lora.shared.scale)
        return L

    def frozen_weights(self, e0, e1, dtype):
        """Int4Experts.weights / BF16Experts.weights (smel/moe.py:25-26, 46-49) in the compute dtype."""
        if not self.int4:
            return self.frozen["gate_up"][e0:e1].to(dtype), self.frozen["down"][e0:e1].to(dtype)
        gu, dn = self.frozen["gate_up"], self.frozen["down"]
        w_gu = dequant_int4(gu["q"][e0:e1], gu["scale"][e0:e1], gu["zero"][e0:e1], self.deq_dtype)
        w_dn = dequant_int4(dn["q"][e0:e1], dn["scale"][e0:e1], dn["zero"][e0:e1], self.deq_dtype)
        return w_gu.to(dtype), w_dn.to(dtype)


# ------------------------------------------------------------------------------------------- experts (A4-A6, A10)


def _grouped_matmul(x, w, counts, transpose_w=True):
    """The CPU branch of ``_gmm`` (smel/moe.py:58-72): per-expert loop over contiguous row groups."""
    outs, s = [], 0
    n = w.shape[1] if transpose_w else w.shape[2]
    for e, c in enumerate(counts):
        if c:
            outs.append(x[s:s + c] @ (w[e].t() if transpose_w else w[e]))
            s += c
    return torch.cat(outs) if outs else x.new_zeros(0, n)


def _expert_groups(counts, group):
    """smel/moe.py:75-85."""
    row = 0
    for e0 in range(0, len(counts), group):
        e1 = min(len(counts), e0 + group)
        sub = counts[e0:e1]
        n = sum(sub)
        if n:
            yield e0, e1, row, row + n, sub
        row += n


class _FrozenExperts(torch.autograd.Function):
    """smel/moe.py:110-143: forward per expert group (dequant, gate_up GEMM, act*up, down GEMM); backward
    re-dequantizes each group and recomputes h, keeps only xs."""

    @staticmethod
    def forward(ctx, xs, counts, layer, dtype):
        ctx.save_for_backward(xs)
        ctx.counts, ctx.layer, ctx.dtype = counts, layer, dtype
        out = xs.new_empty(xs.shape)
        for e0, e1, r0, r1, sub in _expert_groups(counts, layer.expert_group):
            gu, dn = layer.frozen_weights(e0, e1, dtype)
            g, u = _grouped_matmul(xs[r0:r1], gu, sub).chunk(2, dim=-1)
            out[r0:r1] = _grouped_matmul(act(g, layer.act) * u, dn, sub)
        return out

    @staticmethod
    def backward(ctx, dy):
        (xs,) = ctx.saved_tensors
        layer = ctx.layer
        dx = torch.zeros_like(xs)
        dy = dy.to(xs.dtype)
        for e0, e1, r0, r1, sub in _expert_groups(ctx.counts, layer.expert_group):
            gu, dn = layer.frozen_weights(e0, e1, ctx.dtype)
            g, u = _grouped_matmul(xs[r0:r1], gu, sub).chunk(2, dim=-1)
            da = _grouped_matmul(dy[r0:r1], dn, sub, transpose_w=False)
            a, da_dg = act_and_grad(g, layer.act)
            dh = torch.cat([da * u * da_dg, da * a], dim=-1)
            dx[r0:r1] = _grouped_matmul(dh, gu, sub, transpose_w=False)
        return dx, None, None, None


def _selected_expert(x, gu, dn, lora, j, scale, act_name):
    """smel/moe.py:204-211."""
    if lora is None:
        g, u = (x @ gu.t()).chunk(2, dim=-1)
        return (act(g, act_name) * u) @ dn.t()
    g, u = lora_gate_up(x, gu, lora["A_gate"][j], lora["B_gate"][j], lora["A_up"][j], lora["B_up"][j], scale)
    return lora_linear(act(g, act_name) * u, dn, lora["A_down"][j], lora["B_down"][j], scale)


def routed_experts(x2d, topv, topi, layer: OracleLayer, lora: dict | None = None, dtype=torch.float32):
    """smel/moe.py:214-252: stable-argsort dispatch, frozen experts through the recompute Function, selected bf16
    experts (+LoRA) in a loop, scatter to sorted order, undo the sort and sum the K weighted outputs in fp32 (the
    accumulation dtype is ``dtype`` when that is wider)."""
    N, H = x2d.shape
    K = topi.shape[1]
    order, tok, counts_t, _, inv = dispatch_fast(topi, layer.E)
    xs = x2d[tok]
    counts = counts_t.tolist()
    sel = set(int(e) for e in layer.sel_ids)
    rows, vals = [], []
    e_sorted = topi.reshape(-1)[order]
    is_sel = torch.tensor([int(e) in sel for e in e_sorted.tolist()], dtype=torch.bool)
    counts_f = [0 if e in sel else c for e, c in enumerate(counts)]
    fr = (~is_sel).nonzero().squeeze(1)
    if fr.numel():
        rows.append(fr)
        vals.append(_FrozenExperts.apply(xs[fr], counts_f, layer, dtype))
    starts = [sum(counts[:e]) for e in range(len(counts))]
    for j, e in enumerate(layer.sel_ids):
        e = int(e)
        c = counts[e]
        if c == 0:
            continue
        r0 = starts[e]
        rows.append(torch.arange(r0, r0 + c))
        vals.append(_selected_expert(xs[r0:r0 + c], layer.sel_gate_up[j].to(dtype), layer.sel_down[j].to(dtype),
                                     lora, j, layer.ex_scale, layer.act).to(x2d.dtype))
    y = x2d.new_zeros(xs.shape[0], H).index_put((torch.cat(rows),), torch.cat(vals))
    y = y[inv].view(N, K, H)
    acc = torch.promote_types(torch.float32, dtype)
    return (y.to(acc) * topv.to(acc).unsqueeze(-1)).sum(1).to(x2d.dtype)


def shared_mlp(x, layer: OracleLayer, lora: dict | None = None, dtype=torch.float32):
    """smel/moe.py:197-201: gated shared expert with LoRA, times sigmoid(x w_sg^T)."""
    sh = layer.shared
    y = mlp_lora(x, sh["gate_up"].to(dtype), sh["down"].to(dtype), lora, layer.sh_scale, "silu")
    return y * torch.sigmoid(F.linear(x, sh["gate_w"].to(dtype)))


def moe_forward(x2d, layer: OracleLayer, top_k: int, stats=None, forced_topi=None, dtype=None):
    """smel/moe.py:255-263: route -> stats hook -> routed experts + shared expert. ``forced_topi`` replaces the
    router's choice of experts while keeping topv differentiable through the router softmax, as the reference's
    tests force routing (tests/helpers.py:89-106). Computes in x2d's dtype unless ``dtype`` is given."""
    dtype = dtype or x2d.dtype
    x = x2d.to(dtype)
    logits = F.linear(x, layer.gate_w.to(dtype))
    probs, topv, topi = route(x, layer.gate_w.to(dtype), top_k, logits=logits)
    if forced_topi is not None:
        topi = forced_topi.long()
        top = probs.gather(1, topi)
        topv = (top / top.sum(-1, keepdim=True)).to(logits.dtype)
    if stats is not None:
        stats(probs, topv, topi)
    out = routed_experts(x, topv, topi, layer, layer.ex_lora, dtype)
    if layer.shared is not None:
        out = out + shared_mlp(x, layer, layer.sh_lora, dtype)
    return out


def moe_forward_bruteforce(x2d, layer: OracleLayer, topi, dtype=torch.float64):
    """Per-token, per-slot evaluation of the same layer (no dispatch, no grouping): the independent formula the
    composite path is checked against. topv comes from the router softmax at the given ids."""
    x = x2d.to(dtype)
    probs = torch.softmax(F.linear(x, layer.gate_w.to(dtype)), dim=-1)
    T, H = x.shape
    out = torch.zeros(T, H, dtype=dtype)
    sel = {int(e): j for j, e in enumerate(layer.sel_ids)}
    gu_all, dn_all = layer.frozen_weights(0, layer.E, dtype)
    for t in range(T):
        ids = topi[t].tolist()
        w = probs[t, ids]
        w = w / w.sum()
        for k, e in enumerate(ids):
            xt = x[t:t + 1]
            if e in sel:
                y = _selected_expert(xt, layer.sel_gate_up[sel[e]].to(dtype), layer.sel_down[sel[e]].to(dtype),
                                     layer.ex_lora, sel[e], layer.ex_scale, layer.act)
            else:
                g, u = (xt @ gu_all[e].t()).chunk(2, dim=-1)
                y = (act(g, layer.act) * u) @ dn_all[e].t()
            out[t] += w[k] * y[0]
    if layer.shared is not None:
        out = out + shared_mlp(x, layer, layer.sh_lora, dtype)
    return out


def moe_forward_backward(x2d, layer: OracleLayer, top_k, gy, forced_topi=None, dtype=torch.float32):
    """Forward with autograd + backward (the metric's unit of work). Returns (y, dx, {name: grad}) where the LoRA
    gradients are keyed ``ex_<A|B>_<proj>`` / ``sh_<A|B>_<proj>``; LoRA tensors of ``layer`` are used as leaves."""
    x = x2d.to(dtype).clone().requires_grad_(True)
    leaves = {}
    saved = (layer.ex_lora, layer.sh_lora)
    for tag in ("ex", "sh"):
        L = getattr(layer, tag + "_lora")
        if L is None:
            continue
        new = {k: v.detach().to(dtype).clone().requires_grad_(True) for k, v in L.items()}
        for k, v in new.items():
            leaves[f"{tag}_{k}"] = v
        setattr(layer, tag + "_lora", new)
    try:
        y = moe_forward(x, layer, top_k, forced_topi=forced_topi, dtype=dtype)
        y.backward(gy.to(dtype))
    finally:
        layer.ex_lora, layer.sh_lora = saved
    return y.detach(), x.grad.detach(), {k: v.grad.detach() if v.grad is not None else torch.zeros_like(v)
                                         for k, v in leaves.items()}


# ------------------------------------------------------------------------------------ Gemma 4 MoE block (C4)

GEMMA4_NORMS = ("post_attention_layernorm", "pre_feedforward_layernorm", "post_feedforward_layernorm_1",
                "pre_feedforward_layernorm_2", "post_feedforward_layernorm_2", "post_feedforward_layernorm")


def gemma4_moe_block(h, a, W: dict, layer: OracleLayer, top_k: int, eps: float, forced_topi=None,
                     dtype=torch.float32):
    """The Gemma 4 decoder layer from the attention output on (smel/layer_runner.py:243-262): the residual add with
    the post-attention norm, the pre-feed-forward norm, the dense GeGLU MLP with the layer's shared LoRA
    (smel/moe.py:183-194) and its post norm, route_gemma4 on the residual stream, the experts on their own pre norm
    and their post norm, the final norm of the sum, the residual add and the layer scalar. Every norm is the
    reference's torch RMSNorm with a plain weight (plus_one=False). h: residual stream, a: attention output.
    Returns (out, (probs, topv, topi))."""
    from .norm_ref import torch_rmsnorm

    wt = lambda k: W[k].to(dtype)
    rn = lambda x, name: torch_rmsnorm(x, wt(name + ".weight"), eps, plus_one=False)
    h = h.to(dtype)
    h2 = h + rn(a.to(dtype), "post_attention_layernorm")
    xm = rn(h2, "pre_feedforward_layernorm")
    gu = W.get("mlp.gate_up_proj.weight")
    if gu is None:
        gu = torch.cat((W["mlp.gate_proj.weight"], W["mlp.up_proj.weight"]))
    m = mlp_lora(xm, gu.to(dtype), wt("mlp.down_proj.weight"), layer.sh_lora, layer.sh_scale, layer.act)
    m = rn(m, "post_feedforward_layernorm_1")
    rw = {k: wt(k) for k in ("router.scale", "router.proj.weight", "router.per_expert_scale")}
    probs, topv, topi = route_gemma4(h2, rw, top_k, eps, forced_topi)
    e = routed_experts(rn(h2, "pre_feedforward_layernorm_2"), topv, topi, layer, layer.ex_lora, dtype)
    e = rn(e, "post_feedforward_layernorm_2")
    out = (h2 + rn(m + e, "post_feedforward_layernorm")) * wt("layer_scalar")
    return out, (probs, topv, topi)


def gemma4_block_forward_backward(h, a, W: dict, layer: OracleLayer, top_k, eps, gy, forced_topi=None,
                                  dtype=torch.float32):
    """Forward with autograd + backward of :func:`gemma4_moe_block`. Returns (out, dh, da, {name: grad}) with the
    LoRA gradients keyed ``ex_*`` (experts) and ``sh_*`` (the dense MLP)."""
    hh = h.to(dtype).clone().requires_grad_(True)
    aa = a.to(dtype).clone().requires_grad_(True)
    leaves = {}
    saved = (layer.ex_lora, layer.sh_lora)
    for tag in ("ex", "sh"):
        L = getattr(layer, tag + "_lora")
        if L is None:
            continue
        new = {k: v.detach().to(dtype).clone().requires_grad_(True) for k, v in L.items()}
        leaves.update({f"{tag}_{k}": v for k, v in new.items()})
        setattr(layer, tag + "_lora", new)
    try:
        out, _ = gemma4_moe_block(hh, aa, W, layer, top_k, eps, forced_topi, dtype)
        out.backward(gy.to(dtype))
    finally:
        layer.ex_lora, layer.sh_lora = saved
    return out.detach(), hh.grad.detach(), aa.grad.detach(), {
        k: v.grad.detach() if v.grad is not None else torch.zeros_like(v) for k, v in leaves.items()}


# --------------------------------------------------------------------------------------- synthetic layers (C1-C5)


def make_layer(T, H, E, I, K, n_sel=0, r=16, alpha=32.0, shared_inter=None, group=64, down_group=None,
               int4=True, seed=0, sel_ids=None, act_name="silu", lora_b_std=0.02, dtype=torch.bfloat16,
               router_std=0.02, r_shared=None):
    """Synthetic MoE layer of the given shape (the benchmark configs): weights ~N(0, 0.02) in ``dtype``, router
    ~N(0, router_std), frozen experts quantized with :func:`quantize_int4`, selected ids spread as the reference's
    layer benchmark picks them (scripts/bench/bench_layer.py:70) unless given, LoRA A ~ U(+-1/sqrt(in)) and
    B ~ N(0, lora_b_std), rank r (the shared MLP's r_shared when given; scale alpha / rank). Returns
    (x [T,H], OracleLayer)."""
    g = torch.Generator().manual_seed(seed)

    def rnd(*s, std=0.02):
        return (torch.randn(*s, generator=g) * std).to(dtype)

    x = torch.randn(T, H, generator=g).to(dtype)
    gate_w = rnd(E, H, std=router_std)
    gu, dn = rnd(E, 2 * I, H), rnd(E, H, I)
    if int4:
        frozen = {"gate_up": quantize_int4(gu, group), "down": quantize_int4(dn, down_group or min(group, I))}
    else:
        frozen = {"gate_up": gu, "down": dn}
    if sel_ids is None:
        sel_ids = list(range(0, E, max(1, E // n_sel)))[:n_sel] if n_sel else []
    sel_ids = list(sel_ids)
    ids = torch.tensor(sel_ids, dtype=torch.long)
    layer = OracleLayer(gate_w=gate_w, frozen=frozen, int4=int4, sel_ids=sel_ids, act=act_name,
                        deq_dtype=torch.bfloat16)

    def lora_set(k, inter, lead, r=r):
        shp = (lambda *s: (k, *s)) if lead else (lambda *s: s)
        out = {}
        for n, s, fan in (("A_gate", shp(r, H), H), ("A_up", shp(r, H), H), ("A_down", shp(r, inter), inter)):
            out[n] = (torch.rand(*s, generator=g) * 2 - 1) / math.sqrt(fan)
        for n, s in (("B_gate", shp(inter, r)), ("B_up", shp(inter, r)), ("B_down", shp(H, r))):
            out[n] = torch.randn(*s, generator=g) * lora_b_std
        return out

    if sel_ids:
        layer.sel_gate_up, layer.sel_down = gu[ids].clone(), dn[ids].clone()
        layer.ex_lora = lora_set(len(sel_ids), I, True) if r else None
        layer.ex_scale = alpha / r if r else 0.0
    if shared_inter:
        layer.shared = {"gate_up": rnd(2 * shared_inter, H), "down": rnd(H, shared_inter),
                        "gate_w": rnd(1, H)}
        rs = r if r_shared is None else r_shared
        layer.sh_lora = lora_set(0, shared_inter, False, rs) if rs else None
        layer.sh_scale = alpha / rs if rs else 0.0
    return x, layer


def np_seed_inputs(shape, seed):
    """Seeded N(0,1) fp32 numpy array (helper for the integer-path fixtures)."""
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)
