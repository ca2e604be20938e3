"""fp32 path of the MoE layer: the reference's layer run on fp32 tensors (its fp32 models, whose ``_gmm`` falls to a
per-group matmul loop for any non-bf16 tensor, smel/moe.py:58-72, and whose own tests compare at 1e-5,
tests/test_moe.py:10-36). ``smel.moe`` enters it when the activations are float32; the functions keep the reference's
arguments and results.

Every product is an fp32 MFMA of libsmel_moe.so (``smel_gmm_f32`` over the dispatch's tile list, ``smel_wgrad_f32``
for the LoRA weight gradients) and every element-wise step a HIP kernel of the same library (include/smel_f32.h). The
structure follows the reference's composition: route -> stats -> routed experts (dispatch, gather, gate_up with the
LoRA terms added as ``addmm(base, xa, B^T, alpha=s)``, act(g) u, down with its LoRA term, combine) -> shared expert
(``mlp_lora``) times its sigmoid gate, added to the routed output. int4 banks are dequantized to fp32 inside the GEMM
(``q s + z``, the reference's fp32 ``dequant_int4``); a bank whose dtype is bf16 rounds the dequantized weight to
bf16 first, as the reference's dequant to that dtype does.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib as L

M_TILE = 64    # rows per tile of the fp32 GEMMs' tile lists
_ACT = {"silu": 0, "gelu_tanh": 1}
_NAMES = ("A_gate", "B_gate", "A_up", "B_up", "A_down", "B_down")


def f32(t: torch.Tensor, what: str = "tensor") -> torch.Tensor:
    if t.dtype != torch.float32:
        raise TypeError(f"the fp32 path takes float32 tensors; {what} is {t.dtype}")
    return t.contiguous()


def _act_id(name: str) -> int:
    if name not in _ACT:
        raise ValueError(f"unknown activation {name}")
    return _ACT[name]


# ------------------------------------------------------------------------------------------------ weight sets


def _ws(R: int, C: int, kinds: int, **ptrs) -> L.WSetF32:
    w = L.WSetF32()
    w.R, w.C, w.kinds = int(R), int(C), int(kinds)
    for k, v in ptrs.items():
        setattr(w, k, v)
    return w


def _dense(t: torch.Tensor) -> L.WSetF32:
    """One fp32 matrix [R][C] as the shared-kind weight of a dense launch."""
    return _ws(t.shape[0], t.shape[1], 1 << L.KIND_SHARED, wsh=L.ptr(t))


def _sel(t: torch.Tensor) -> L.WSetF32:
    """A stack [n][R][C] of per-slot fp32 matrices (selected experts or their LoRA factors), selected tiles only."""
    return _ws(t.shape[1], t.shape[2], 1 << L.KIND_SEL, wsel=L.ptr(t))


def bank_wset(bank, which: str, sel: torch.Tensor | None = None) -> L.WSetF32:
    """gate_up ('gu') or down ('dn') of a frozen bank, plus the selected experts' fp32 copies when given."""
    from .moe import Int4Experts
    if isinstance(bank, Int4Experts):
        d = bank.gu if which == "gu" else bank.dn
        q, s, z = d["q"], d["scale"], d["zero"]
        if s.dtype != torch.bfloat16 or z.dtype != torch.bfloat16 or q.dtype != torch.uint8:
            raise TypeError("Int4Experts: q must be uint8 and scale / zero bfloat16 (the quantize_int4 format)")
        E, R, Ch = q.shape
        C = 2 * Ch
        w = _ws(R, C, 1 << L.KIND_INT4, q4=L.ptr(q), scale=L.ptr(s), zero=L.ptr(z))
        w.group = C // s.shape[-1]
        w.q4_round_bf16 = int(bank.dtype == torch.bfloat16)
    else:
        t = f32(bank.gate_up if which == "gu" else bank.down, "the frozen bank")
        w = _ws(t.shape[1], t.shape[2], 1 << L.KIND_BF16, wf=L.ptr(t))
        w._keep = t   # a contiguous copy lives as long as the weight set that points into it
    if sel is not None:
        w.wsel = L.ptr(sel)
        w.kinds |= 1 << L.KIND_SEL
    return w


# ------------------------------------------------------------------------------------------------ launches


def gmm(w: L.WSetF32, trans: int, tl, A: torch.Tensor, lda: int, C: torch.Tensor, ldc: int, alpha: float = 1.0,
        beta: float = 0.0, gkind=None, tag: str = "gemm_f32"):
    """smel_gmm_f32 over the tile list tl = (tiles, n_tiles, max_tiles)."""
    tiles, ntiles, maxt = tl
    L.call("smel_gmm_f32", ctypes.byref(w), int(trans), L.ptr(gkind), L.ptr(tiles), L.ptr(ntiles), int(maxt),
           L.ptr(A), int(lda), float(alpha), float(beta), L.ptr(C), int(ldc), L.stream(), tag=tag)


def wgrad(X, ldx: int, Y, ldy: int, offsets, jobs, n_jobs: int, M: int, N: int, alpha: float, out, tag="wgrad_f32"):
    """out[j] = alpha X_j^T Y_j over the rows of job j's group."""
    L.call("smel_wgrad_f32", L.ptr(X), int(ldx), L.ptr(Y), int(ldy), L.ptr(offsets), L.ptr(jobs), int(n_jobs), int(M),
           int(N), float(alpha), L.ptr(out), int(M * N), L.stream(), tag=tag)


_dense_cache = {}


def dense_tiles(T: int, device):
    """Tile list of one dense group of T rows (group 0, shared kind) and its row offsets [0, T]."""
    key = (T, str(device))
    if key not in _dense_cache:
        n = (T + M_TILE - 1) // M_TILE
        tl = [(0, r, min(T, r + M_TILE), L.KIND_SHARED << 16) for r in range(0, T, M_TILE)] or [(0, 0, 0, 0)]
        t = torch.tensor(tl, dtype=torch.int32).reshape(-1).to(device)
        offs = torch.tensor([0, T], dtype=torch.int32, device=device)
        _dense_cache[key] = ((t, torch.tensor([n], dtype=torch.int32, device=device), n), offs,
                             torch.zeros(1, dtype=torch.int32, device=device))
    return _dense_cache[key]


def count_tiles(counts: list, kind: int, device):
    """Tile list of 64-row tiles over contiguous row groups of the given host sizes (group e = matrix e of the given
    kind, carried in each tile), and the groups' row offsets."""
    tl, offs, row = [], [0], 0
    for e, c in enumerate(counts):
        for r0 in range(row, row + c, M_TILE):
            tl.append((e, r0, min(row + c, r0 + M_TILE), (kind << 16) | e))
        row += c
        offs.append(row)
    n = len(tl)
    t = torch.tensor(tl or [(0, 0, 0, 0)], dtype=torch.int32).reshape(-1).to(device)
    return (t, torch.tensor([n], dtype=torch.int32).to(device), n), torch.tensor(offs, dtype=torch.int32).to(device)


def _lora_f32(lora):
    """The six factors of a LoRA set as fp32 contiguous tensors (the reference casts them to the activations'
    dtype), and its scale."""
    return {n: getattr(lora, n).detach().float().contiguous() for n in _NAMES}, float(lora.scale)


def _grad_like(lora, grads: dict):
    return [grads.get(n).to(getattr(lora, n).dtype) if getattr(lora, n).requires_grad else None for n in _NAMES]


# ------------------------------------------------------------------------------------------------ gated MLP core


class _Saved:
    __slots__ = ("x", "h", "a", "xa_g", "xa_u", "xa_d")


def mlp_core_fwd(x, tl, I: int, w_gu, w_dn, gu_split, lora_w, s: float, lora_w_sel: bool, act: int, need: bool,
                 tag: str = "f32"):
    """The gated MLP over the rows of the tile list: h = [g | u] = x W_gu^T (+ s (x A_g^T) B_g^T, + s (x A_u^T) B_u^T),
    a = act(g) u, y = a W_dn^T (+ s (a A_d^T) B_d^T). ``w_gu`` is one weight set of 2I rows, or None with
    ``gu_split`` = (gate, up) weight sets of I rows each. ``lora_w`` = dict of fp32 factors (stacked per slot when
    ``lora_w_sel``) or None. ``tag`` names the launches for timing. Returns (y, saved)."""
    M, H = x.shape
    dev = x.device
    e = lambda *sh: torch.empty(*sh, dtype=torch.float32, device=dev)
    h = e(M, 2 * I)
    if w_gu is not None:
        gmm(w_gu, 0, tl, x, H, h, 2 * I, tag=f"gemm_{tag}_gu")
    else:
        gmm(gu_split[0], 0, tl, x, H, h, 2 * I, tag=f"gemm_{tag}_gu")
        gmm(gu_split[1], 0, tl, x, H, h[:, I:], 2 * I, tag=f"gemm_{tag}_gu")
    sv = _Saved()
    sv.xa_g = sv.xa_u = sv.xa_d = None
    wl = _sel if lora_w_sel else (lambda t: _dense(t))
    if lora_w is not None:
        r = lora_w["A_gate"].shape[-2]
        sv.xa_g, sv.xa_u = e(M, r), e(M, r)
        gmm(wl(lora_w["A_gate"]), 0, tl, x, H, sv.xa_g, r, tag=f"lora_{tag}")
        gmm(wl(lora_w["A_up"]), 0, tl, x, H, sv.xa_u, r, tag=f"lora_{tag}")
        gmm(wl(lora_w["B_gate"]), 0, tl, sv.xa_g, r, h, 2 * I, alpha=s, beta=1.0, tag=f"lora_{tag}")
        gmm(wl(lora_w["B_up"]), 0, tl, sv.xa_u, r, h[:, I:], 2 * I, alpha=s, beta=1.0, tag=f"lora_{tag}")
    a = e(M, I)
    L.call("smel_act_gate_f32", L.ptr(h), 2 * I, M, I, act, L.ptr(a), I, L.stream(), tag=f"act_{tag}")
    Hout = w_dn.R
    y = e(M, Hout)
    gmm(w_dn, 0, tl, a, I, y, Hout, tag=f"gemm_{tag}_dn")
    if lora_w is not None:
        r = lora_w["A_down"].shape[-2]
        sv.xa_d = e(M, r)
        gmm(wl(lora_w["A_down"]), 0, tl, a, I, sv.xa_d, r, tag=f"lora_{tag}")
        gmm(wl(lora_w["B_down"]), 0, tl, sv.xa_d, r, y, Hout, alpha=s, beta=1.0, tag=f"lora_{tag}")
    if need:
        sv.x, sv.h, sv.a = x, h, a
    return y, sv


def mlp_core_bwd(sv: _Saved, dy, tl, I: int, w_gu, w_dn, gu_split, lora_w, s: float, lora_w_sel: bool, act: int,
                 offsets, jobs, n_jobs: int, want_grads: bool, tag: str = "f32"):
    """Backward of mlp_core_fwd: dx over the tile rows, and the LoRA factor gradients (fp32, stacked per job) when
    ``want_grads``: job j's rows are those of group jobs[j] (offsets)."""
    M, Hout = dy.shape
    H = sv.x.shape[1]
    dev = dy.device
    e = lambda *sh: torch.empty(*sh, dtype=torch.float32, device=dev)
    wl = _sel if lora_w_sel else (lambda t: _dense(t))
    grads = {}
    da = e(M, I)
    gmm(w_dn, 1, tl, dy, Hout, da, I, tag=f"gemm_{tag}_dn_bwd")
    if lora_w is not None:
        r = lora_w["A_down"].shape[-2]
        dz = e(M, r)
        gmm(wl(lora_w["B_down"]), 1, tl, dy, Hout, dz, r, alpha=s, tag=f"lora_{tag}")
        gmm(wl(lora_w["A_down"]), 1, tl, dz, r, da, I, beta=1.0, tag=f"lora_{tag}")
        if want_grads:
            grads["B_down"] = e(n_jobs, Hout, r)
            grads["A_down"] = e(n_jobs, r, I)
            wgrad(dy, Hout, sv.xa_d, r, offsets, jobs, n_jobs, Hout, r, s, grads["B_down"], tag=f"wgrad_{tag}")
            wgrad(dz, r, sv.a, I, offsets, jobs, n_jobs, r, I, 1.0, grads["A_down"], tag=f"wgrad_{tag}")
    dh = e(M, 2 * I)
    L.call("smel_act_gate_bwd_f32", L.ptr(sv.h), 2 * I, L.ptr(da), I, M, I, act, L.ptr(dh), 2 * I, L.stream(),
           tag=f"act_{tag}")
    dx = e(M, H)
    if w_gu is not None:
        gmm(w_gu, 1, tl, dh, 2 * I, dx, H, tag=f"gemm_{tag}_gu_bwd")
    else:
        gmm(gu_split[0], 1, tl, dh, 2 * I, dx, H, tag=f"gemm_{tag}_gu_bwd")
        gmm(gu_split[1], 1, tl, dh[:, I:], 2 * I, dx, H, beta=1.0, tag=f"gemm_{tag}_gu_bwd")
    if lora_w is not None:
        r = lora_w["A_gate"].shape[-2]
        dzg, dzu = e(M, r), e(M, r)
        gmm(wl(lora_w["B_gate"]), 1, tl, dh, 2 * I, dzg, r, alpha=s, tag=f"lora_{tag}")
        gmm(wl(lora_w["B_up"]), 1, tl, dh[:, I:], 2 * I, dzu, r, alpha=s, tag=f"lora_{tag}")
        gmm(wl(lora_w["A_gate"]), 1, tl, dzg, r, dx, H, beta=1.0, tag=f"lora_{tag}")
        gmm(wl(lora_w["A_up"]), 1, tl, dzu, r, dx, H, beta=1.0, tag=f"lora_{tag}")
        if want_grads:
            for n in ("B_gate", "B_up"):
                grads[n] = e(n_jobs, I, r)
            for n in ("A_gate", "A_up"):
                grads[n] = e(n_jobs, r, H)
            wgrad(dh, 2 * I, sv.xa_g, r, offsets, jobs, n_jobs, I, r, s, grads["B_gate"], tag=f"wgrad_{tag}")
            wgrad(dh[:, I:], 2 * I, sv.xa_u, r, offsets, jobs, n_jobs, I, r, s, grads["B_up"], tag=f"wgrad_{tag}")
            wgrad(dzg, r, sv.x, H, offsets, jobs, n_jobs, r, H, 1.0, grads["A_gate"], tag=f"wgrad_{tag}")
            wgrad(dzu, r, sv.x, H, offsets, jobs, n_jobs, r, H, 1.0, grads["A_up"], tag=f"wgrad_{tag}")
    return dx, grads


# ------------------------------------------------------------------------------------------------ router


class RouteFn(torch.autograd.Function):
    """route (smel/moe.py:162-167) on fp32 tensors: logits = x W_r^T (fp32 MFMA), softmax, top-k, renorm; topv fp32
    (the logits' dtype), differentiable w.r.t. x."""

    @staticmethod
    def forward(ctx, x, gate_w, top_k):
        T, H = x.shape
        E = gate_w.shape[0]
        dev = x.device
        tl, _, _ = dense_tiles(T, dev)
        logits = torch.empty(T, E, dtype=torch.float32, device=dev)
        gmm(_dense(gate_w), 0, tl, x, H, logits, E, tag="route_f32")
        probs = torch.empty(T, E, dtype=torch.float32, device=dev)
        topv = torch.empty(T, top_k, dtype=torch.float32, device=dev)
        topi = torch.empty(T, top_k, dtype=torch.int64, device=dev)
        topi32 = torch.empty(T, top_k, dtype=torch.int32, device=dev)
        L.call("smel_route_select_f32", L.ptr(logits), E, T, E, top_k, None, L.ptr(probs), L.ptr(topv), L.ptr(topi),
               L.ptr(topi32), L.stream(), tag="route_f32")
        ctx.save_for_backward(probs, topi32, gate_w)
        ctx.mark_non_differentiable(probs, topi)
        return probs, topv, topi

    @staticmethod
    def backward(ctx, dprobs, dtopv, dtopi):
        if dtopv is None:
            return None, None, None
        probs, topi32, gate_w = ctx.saved_tensors
        return _router_bwd(dtopv, probs, topi32, gate_w, None), None, None


def _router_bwd(dtopv, probs, topi32, w, pes):
    T, E = probs.shape
    K = topi32.shape[1]
    dev = probs.device
    dl = torch.empty(T, E, dtype=torch.float32, device=dev)
    dtv = dtopv.float().contiguous()
    L.call("smel_route_bwd_f32", L.ptr(dtv), L.ptr(probs), L.ptr(topi32), L.ptr(pes), T, K, E, L.ptr(dl), L.stream(),
           tag="route_f32_bwd")
    tl, _, _ = dense_tiles(T, dev)
    dx = torch.empty(T, w.shape[1], dtype=torch.float32, device=dev)
    gmm(_dense(w), 1, tl, dl, E, dx, w.shape[1], tag="route_f32_bwd")
    return dx


class RouteGemma4Fn(torch.autograd.Function):
    """route_gemma4 (smel/moe.py:170-180) on fp32 tensors: weightless RMSNorm of h, x router.scale x fp32(H^-1/2),
    logits, softmax, top-k, renorm, x per_expert_scale; differentiable w.r.t. h."""

    @staticmethod
    def forward(ctx, h, scale, proj, pes, top_k, eps):
        T, H = h.shape
        E = proj.shape[0]
        dev = h.device
        hs = float(torch.tensor(H ** -0.5, dtype=torch.float32))
        xn = torch.empty(T, H, dtype=torch.float32, device=dev)
        rstd = torch.empty(T, dtype=torch.float32, device=dev)
        L.call("smel_route_prenorm_f32", L.ptr(h), L.ptr(scale), T, H, float(eps), hs, L.ptr(xn), L.ptr(rstd),
               L.stream(), tag="route_f32")
        tl, _, _ = dense_tiles(T, dev)
        logits = torch.empty(T, E, dtype=torch.float32, device=dev)
        gmm(_dense(proj), 0, tl, xn, H, logits, E, tag="route_f32")
        probs = torch.empty(T, E, dtype=torch.float32, device=dev)
        topv = torch.empty(T, top_k, dtype=torch.float32, device=dev)
        topi = torch.empty(T, top_k, dtype=torch.int64, device=dev)
        topi32 = torch.empty(T, top_k, dtype=torch.int32, device=dev)
        L.call("smel_route_select_f32", L.ptr(logits), E, T, E, top_k, L.ptr(pes), L.ptr(probs), L.ptr(topv),
               L.ptr(topi), L.ptr(topi32), L.stream(), tag="route_f32")
        ctx.save_for_backward(h, scale, proj, pes, probs, topi32, rstd)
        ctx.hs = hs
        ctx.mark_non_differentiable(probs, topi)
        return probs, topv, topi

    @staticmethod
    def backward(ctx, dprobs, dtopv, dtopi):
        if dtopv is None:
            return None, None, None, None, None, None
        h, scale, proj, pes, probs, topi32, rstd = ctx.saved_tensors
        T, H = h.shape
        dxn = _router_bwd(dtopv, probs, topi32, proj, pes)
        dh = torch.empty(T, H, dtype=torch.float32, device=h.device)
        L.call("smel_route_prenorm_bwd_f32", L.ptr(h), L.ptr(scale), L.ptr(rstd), L.ptr(dxn), T, H, ctx.hs, L.ptr(dh),
               L.stream(), tag="route_f32_bwd")
        return dh, None, None, None, None, None


# ------------------------------------------------------------------------------------------------ routed experts


def _sel_stack(t, what):
    return None if t is None else f32(t, what)


class RoutedFn(torch.autograd.Function):
    """routed_experts (smel/moe.py:214-252) on fp32 tensors: dispatch (the stable counting sort of smel_dispatch,
    64-row tiles), the gathered rows xs = x[order // K], the frozen and selected experts' gated MLP over the grouped
    tiles (the selected experts' LoRA on their tiles only), and the fixed-order combine. Differentiable w.r.t. x,
    topv and the expert LoRA factors."""

    @staticmethod
    def forward(ctx, x, topv, topi, ex, lora, record_err, *leaves):
        T, H = x.shape
        K = topi.shape[1]
        E = ex.E
        TK = T * K
        dev = x.device
        st = L.stream()
        lib = L.load()
        maxt = lib.smel_dispatch_max_tiles(TK, E, 0, M_TILE)
        i32 = lambda *s: torch.empty(*s, dtype=torch.int32, device=dev)
        counts, offsets, order, inv = i32(E), i32(E + 1), i32(max(TK, 1)), i32(max(TK, 1))
        tiles, tiles_g, ntiles, err = i32(maxt * 4), i32(maxt * 4), i32(1), i32(1)
        ws = i32(max(1, lib.smel_dispatch_ws_size(TK, E)))
        gk = ex.gkind(False, dev)
        ids = topi.contiguous()
        L.call("smel_dispatch", L.ptr(ids), int(ids.dtype == torch.int64), T, K, E, 0, M_TILE, L.ptr(gk), L.ptr(counts),
               L.ptr(offsets), L.ptr(order), L.ptr(inv), L.ptr(tiles), L.ptr(tiles_g), L.ptr(ntiles), L.ptr(err), 0,
               None, None, L.ptr(ws), st, tag="dispatch_f32")
        record_err(err)
        tl = (tiles, ntiles, maxt)
        xs = torch.empty(TK, H, dtype=torch.float32, device=dev)
        # rows past offsets[E] (slots the dispatch dropped for an id outside [0, E)) are zero rows
        L.call("smel_gather_rows_f32", L.ptr(x), H, L.ptr(order), K, offsets.data_ptr() + 4 * E, TK, H, L.ptr(xs), st,
               tag="gather_f32")
        has_sel = ex.sel_ids is not None and len(ex._slot) > 0
        sel_gu = _sel_stack(ex.sel_gate_up, "sel_gate_up") if has_sel else None
        sel_dn = _sel_stack(ex.sel_down, "sel_down") if has_sel else None
        w_gu, w_dn = bank_wset(ex.frozen, "gu", sel_gu), bank_wset(ex.frozen, "dn", sel_dn)
        I = w_dn.C
        lw, s = _lora_f32(lora) if (lora is not None and has_sel) else (None, 0.0)
        need = any(ctx.needs_input_grad[i] for i in (0, 1)) or any(ctx.needs_input_grad[6:])
        ys, sv = mlp_core_fwd(xs, tl, I, w_gu, w_dn, None, lw, s, True, _act_id(ex.act), need, tag="f32_ex")
        tv = topv.detach().float().contiguous()
        out = torch.empty(T, H, dtype=torch.float32, device=dev)
        L.call("smel_combine_f32", L.ptr(ys), L.ptr(tv), L.ptr(inv), T, K, H, L.ptr(out), st, tag="combine_f32")
        if need:
            ctx.keep = (sv, ys, tv, inv, offsets, tl, w_gu, w_dn, lw, s, I, (sel_gu, sel_dn), ex, lora, T, K)
            ctx.topv_dtype = topv.dtype
        else:
            ctx.keep = None
        return out

    @staticmethod
    def backward(ctx, dout):
        sv, ys, tv, inv, offsets, tl, w_gu, w_dn, lw, s, I, _hold, ex, lora, T, K = ctx.keep
        ctx.keep = None
        dev = dout.device
        H = ys.shape[1]
        dout = f32(dout, "the output gradient")
        dys = torch.empty_like(ys)
        dtopv = torch.empty(T, K, dtype=torch.float32, device=dev)
        L.call("smel_combine_bwd_f32", L.ptr(ys), L.ptr(dout), L.ptr(tv), L.ptr(inv), T, K, H, L.ptr(dys), L.ptr(dtopv),
               L.stream(), tag="combine_f32")
        jobs = None
        n_jobs = 0
        if lw is not None:
            jobs = ex.sel_ids.to(device=dev, dtype=torch.int32)
            n_jobs = int(jobs.numel())
        dxs, grads = mlp_core_bwd(sv, dys, tl, I, w_gu, w_dn, None, lw, s, True, _act_id(ex.act), offsets, jobs, n_jobs,
                                  lw is not None, tag="f32_ex")
        dx = torch.empty(T, H, dtype=torch.float32, device=dev)
        L.call("smel_dx_reduce_f32", L.ptr(dxs), L.ptr(inv), T, K, H, L.ptr(dx), L.stream(), tag="dx_reduce_f32")
        g = _grad_like(lora, grads) if lw is not None else ([None] * 6 if lora is not None else [])
        return (dx, dtopv.to(ctx.topv_dtype), None, None, None, None, *g)


# ------------------------------------------------------------------------------------------------ dense MLP


class MLPFn(torch.autograd.Function):
    """mlp_lora (smel/moe.py:183-194) on fp32 tensors: the gated MLP as one dense group of the fp32 GEMMs, LoRA on
    all three projections; differentiable w.r.t. x and the LoRA factors."""

    @staticmethod
    def forward(ctx, x, w_gate, w_up, w_down, w_gate_up, lora, act_name, *leaves):
        T, H = x.shape
        dev = x.device
        tl, offs, jobs = dense_tiles(T, dev)
        if w_gate_up is not None:
            w_gu, split = _dense(w_gate_up), None
            I = w_gate_up.shape[0] // 2
        else:
            w_gu, split = None, (_dense(w_gate), _dense(w_up))
            I = w_gate.shape[0]
        w_dn = _dense(w_down)
        lw, s = _lora_f32(lora) if lora is not None else (None, 0.0)
        need = ctx.needs_input_grad[0] or any(ctx.needs_input_grad[7:])
        y, sv = mlp_core_fwd(x, tl, I, w_gu, w_dn, split, lw, s, False, _act_id(act_name), need, tag="f32_mlp")
        ctx.keep = (sv, tl, offs, jobs, I, w_gu, w_dn, split, lw, s, lora, act_name,
                    (w_gate, w_up, w_down, w_gate_up)) if need else None
        return y

    @staticmethod
    def backward(ctx, dy):
        sv, tl, offs, jobs, I, w_gu, w_dn, split, lw, s, lora, act_name, _hold = ctx.keep
        ctx.keep = None
        dy = f32(dy, "the output gradient")
        dx, grads = mlp_core_bwd(sv, dy, tl, I, w_gu, w_dn, split, lw, s, False, _act_id(act_name), offs, jobs, 1,
                                 lw is not None, tag="f32_mlp")
        g = []
        if lora is not None:
            g = [grads[n].reshape(getattr(lora, n).shape).to(getattr(lora, n).dtype)
                 if getattr(lora, n).requires_grad else None for n in _NAMES]
        return (dx, None, None, None, None, None, None, *g)


class GateAddFn(torch.autograd.Function):
    """shared_mlp's gate and moe_forward's sum (smel/moe.py:201, :263) on fp32 tensors: out = base + y sigmoid(x
    w_sg^T) (base optional); differentiable w.r.t. y, x and base."""

    @staticmethod
    def forward(ctx, y, x, w_sg, base):
        T, H = y.shape
        dev = y.device
        tl, _, _ = dense_tiles(T, dev)
        sl = torch.empty(T, 1, dtype=torch.float32, device=dev)
        gmm(_dense(w_sg), 0, tl, x, x.shape[1], sl, 1, tag="gate_f32")
        out = torch.empty(T, H, dtype=torch.float32, device=dev)
        L.call("smel_gate_mul_f32", L.ptr(y), L.ptr(sl), L.ptr(base), T, H, L.ptr(out), L.stream(), tag="gate_f32")
        ctx.save_for_backward(y, sl, w_sg)
        ctx.has_base = base is not None
        return out

    @staticmethod
    def backward(ctx, dout):
        y, sl, w_sg = ctx.saved_tensors
        T, H = y.shape
        dev = y.device
        dout = f32(dout, "the output gradient")
        dy = torch.empty_like(y)
        ds = torch.empty(T, 1, dtype=torch.float32, device=dev)
        L.call("smel_gate_mul_bwd_f32", L.ptr(y), L.ptr(sl), L.ptr(dout), T, H, L.ptr(dy), L.ptr(ds), L.stream(),
               tag="gate_f32")
        tl, _, _ = dense_tiles(T, dev)
        dx = torch.empty(T, w_sg.shape[1], dtype=torch.float32, device=dev)
        gmm(_dense(w_sg), 1, tl, ds, 1, dx, w_sg.shape[1], tag="gate_f32")
        return dy, dx, None, (dout if ctx.has_base else None)


# ------------------------------------------------------------------------------------------------ frozen experts


def frozen_fwd(xs, counts: list, bank, act_name: str):
    """FrozenExpertsFn.forward (smel/moe.py:120-126) on fp32 rows sorted by expert (host counts): the gated MLP of
    each expert over its rows. Returns (out, what the backward needs)."""
    from .moe import Int4Experts
    kind = L.KIND_INT4 if isinstance(bank, Int4Experts) else L.KIND_BF16
    tl, _ = count_tiles(counts, kind, xs.device)
    w_gu, w_dn = bank_wset(bank, "gu"), bank_wset(bank, "dn")
    I = w_dn.C
    y, sv = mlp_core_fwd(xs, tl, I, w_gu, w_dn, None, None, 0.0, False, _act_id(act_name), True, tag="f32_frozen")
    return y, (sv, tl, w_gu, w_dn, I, act_name, bank)


def frozen_bwd(keep, dy):
    """FrozenExpertsFn.backward (smel/moe.py:128-143) on fp32: dX of the rows (no weight gradients)."""
    sv, tl, w_gu, w_dn, I, act_name, _bank = keep
    dx, _ = mlp_core_bwd(sv, f32(dy, "the output gradient"), tl, I, w_gu, w_dn, None, None, 0.0, False,
                         _act_id(act_name), None, None, 0, False, tag="f32_frozen")
    return dx
