"""The fp32 path (float32 activations: the reference's fp32 models, whose _gmm falls to per-group matmuls for any
non-bf16 tensor, smel/moe.py:58-72, and whose own tests compare at 1e-5, tests/test_moe.py:10-36 and
tests/test_layer_major.py:86-134) against the oracle computed in fp64 and the reference's own fp32 golden outputs.

The bar is the reference's fp32 one: ||out - ref|| / ||ref|| <= 1e-5 (rel_err of smel/quant.py:108-110) for outputs,
dX and every LoRA gradient; the measured errors are printed."""
import itertools

import pytest
import torch

from helpers import LORA_NAMES, c1_layer, to_device_layer
from oracle import moe_ref as R

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-5


def _say(msg):
    print(msg, flush=True)


def _check(out, ref, name, tol=TOL):
    e = R.rel_err(out.detach().cpu(), ref.detach().cpu())
    _say(f"  {name}: rel {e:.2e}")
    assert e <= tol, f"{name}: rel {e:.3e} > {tol}"
    return e


# ------------------------------------------------------------------------------------------------ GEMM primitives


def _int4_bank(E, R_, C, group, seed):
    g = torch.Generator().manual_seed(seed)
    return R.quantize_int4(torch.randn(E, R_, C, generator=g) * 0.05, group)


@pytest.mark.parametrize("pad", [0, 3])
@pytest.mark.parametrize("trans", [0, 1])
@pytest.mark.parametrize("kind", ["int4", "fp32", "sel", "int4_bf16"])
def test_gmm_f32_against_fp64(trans, kind, pad):
    """smel_gmm_f32 on a tile list of uneven groups (an empty one, one longer than a tile, rows not a multiple of 64,
    K not a multiple of 16, N not a multiple of 64), each weight kind, both orientations, with beta = 1 on top of a
    given C, against the fp64 per-group product."""
    from smel import _lib as L
    from smel import moe_f32 as F
    _say(f"gmm_f32 trans={trans} kind={kind} pad={pad}")
    torch.manual_seed(1)
    E, Rw, Cw, group = 5, 96, 136, 8     # one matrix [96][136]
    counts = [70, 0, 5, 130, 33]
    rows = sum(counts)
    q = _int4_bank(E, Rw, Cw, group, 3)
    if kind.startswith("int4"):
        deq = R.dequant_int4(q["q"], q["scale"], q["zero"], torch.bfloat16 if kind == "int4_bf16" else torch.float32)
        W = deq.double()
    else:
        Wf = torch.randn(E, Rw, Cw) * 0.05
        W = Wf.double()
    K, N = (Rw, Cw) if trans else (Cw, Rw)
    lda = K + pad                         # pad 3: not a multiple of 4, the scalar load path
    A = torch.randn(rows, lda)
    C0 = torch.randn(rows, N + 5)
    kconst = {"int4": L.KIND_INT4, "int4_bf16": L.KIND_INT4, "fp32": L.KIND_BF16, "sel": L.KIND_SEL}[kind]
    tl, _ = F.count_tiles(counts, kconst, DEV)
    if kind.startswith("int4"):
        dq = {k: v.to(DEV) for k, v in q.items()}
        w = F._ws(Rw, Cw, 1 << L.KIND_INT4, q4=L.ptr(dq["q"]), scale=L.ptr(dq["scale"]), zero=L.ptr(dq["zero"]))
        w.group = group
        w.q4_round_bf16 = int(kind == "int4_bf16")
    elif kind == "fp32":
        Wd = Wf.to(DEV)
        w = F._ws(Rw, Cw, 1 << L.KIND_BF16, wf=L.ptr(Wd))
    else:
        Wd = Wf.to(DEV)
        w = F._ws(Rw, Cw, 1 << L.KIND_SEL, wsel=L.ptr(Wd))
    Ad, Cd = A.to(DEV), C0.to(DEV)
    F.gmm(w, trans, tl, Ad, lda, Cd, N + 5, alpha=0.75, beta=1.0)
    torch.cuda.synchronize()
    ref = C0.double().clone()
    r = 0
    for e, c in enumerate(counts):
        We = W[e] if trans else W[e].t()
        ref[r:r + c, :N] += 0.75 * (A[r:r + c, :K].double() @ We)
        r += c
    _check(Cd.cpu(), ref, "C", tol=1e-6)


def test_wgrad_f32_against_fp64():
    """smel_wgrad_f32: per job, alpha X^T Y over its group's rows (an empty group writes zeros; M, N not multiples of
    64; rows not multiples of 16), against fp64."""
    from smel import moe_f32 as F
    _say("wgrad_f32")
    torch.manual_seed(2)
    counts = [37, 0, 200, 5]
    offs = torch.tensor([0] + list(itertools.accumulate(counts)), dtype=torch.int32)
    rows, M, N = sum(counts), 40, 136
    X, Y = torch.randn(rows, M + 4), torch.randn(rows, N)
    jobs = torch.tensor([2, 1, 0, 3], dtype=torch.int32)
    out = torch.full((4, M, N), float("nan"), device=DEV)
    Xd, Yd, od, jd = X.to(DEV), Y.to(DEV), offs.to(DEV), jobs.to(DEV)
    F.wgrad(Xd, M + 4, Yd, N, od, jd, 4, M, N, 0.5, out)
    torch.cuda.synchronize()
    for j, g in enumerate(jobs.tolist()):
        r0, r1 = int(offs[g]), int(offs[g + 1])
        ref = 0.5 * X[r0:r1, :M].double().t() @ Y[r0:r1].double()
        if r1 == r0:
            assert torch.equal(out[j].cpu(), torch.zeros(M, N))
        else:
            _check(out[j].cpu(), ref, f"job {j} (group {g})", tol=1e-6)


# ------------------------------------------------------------------------------------------------ router


@pytest.mark.parametrize("E", [8, 64, 256, 300])
def test_route_select_f32_given_logits(E):
    """Selection from given fp32 logits against torch on the CPU (fp32 softmax, top-k, renorm): the ids exactly
    (lower id first among equal probabilities, planted ties included), probs and topv to an fp32 ulp or two."""
    from smel import _lib as L
    _say(f"route_select_f32 E={E}")
    torch.manual_seed(E)
    T, K = 300, min(8, E)
    lg = torch.randn(T, E) * 2
    lg[:20, 5] = lg[:20, 3]               # ties: equal logits give equal probabilities
    lg[20:40, :] = 0.25
    probs = torch.empty(T, E, device=DEV)
    topv = torch.empty(T, K, device=DEV)
    topi = torch.empty(T, K, dtype=torch.int64, device=DEV)
    topi32 = torch.empty(T, K, dtype=torch.int32, device=DEV)
    lgd = lg.to(DEV)
    L.call("smel_route_select_f32", L.ptr(lgd), E, T, E, K, None, L.ptr(probs), L.ptr(topv), L.ptr(topi),
           L.ptr(topi32), L.stream())
    torch.cuda.synchronize()
    p_ref = torch.softmax(lg, -1)
    _, i_ref = R.topk_lowest_index(probs.cpu(), K)   # the tie rule on the kernel's own probabilities
    assert torch.equal(topi.cpu(), i_ref) and torch.equal(topi32.cpu().long(), i_ref)
    assert torch.allclose(probs.cpu(), p_ref, rtol=1e-6, atol=1e-9)
    v_ref, i_cpu = R.topk_lowest_index(p_ref, K)
    assert torch.equal(i_cpu, i_ref)
    assert torch.allclose(topv.cpu(), v_ref / v_ref.sum(-1, keepdim=True), rtol=1e-6, atol=1e-9)


def test_route_f32_api_forward_backward():
    """route() on fp32 tensors: probs / topv against fp64, the ids equal to those of the fp64 router (no near-ties
    at this size), dX through topv against fp64 autograd of the reference formula."""
    from smel.moe import route
    _say("route fp32 API")
    torch.manual_seed(5)
    T, H, E, K = 512, 256, 64, 8
    x = torch.randn(T, H)
    w = torch.randn(E, H) * 0.05
    xd = x.to(DEV).requires_grad_(True)
    probs, topv, topi = route(xd, w.to(DEV), K)
    assert topv.dtype == torch.float32 and probs.dtype == torch.float32 and topi.dtype == torch.int64
    gy = torch.randn(T, K)
    (topv * gy.to(DEV)).sum().backward()
    x64 = x.double().requires_grad_(True)
    p64, v64, i64 = R.route(x64, w.double(), K)
    assert torch.equal(topi.cpu(), i64)
    _check(probs.cpu(), p64, "probs")
    _check(topv.cpu(), v64, "topv")
    (v64 * gy.double()).sum().backward()
    _check(xd.grad.cpu(), x64.grad, "dx")


def test_route_gemma4_f32_forward_backward(golden_c1):
    """route_gemma4 on fp32 tensors: the reference's golden fp32 probs / topv / ids on the C1 input, and dH through
    topv against fp64 autograd of the reference formula."""
    from smel.moe import route_gemma4
    _say("route_gemma4 fp32")
    t = golden_c1
    W = {k[len("gemma."):]: v for k, v in t.items() if k.startswith("gemma.router")}
    h = t["in.x"].to(DEV).requires_grad_(True)
    probs, topv, topi = route_gemma4(h, {k: v.to(DEV) for k, v in W.items()}, 2, 1e-6)
    assert torch.equal(topi.cpu(), t["gemma.topi"])
    _check(probs.cpu(), t["gemma.probs"], "probs vs golden")
    _check(topv.cpu(), t["gemma.topv"], "topv vs golden")
    gy = torch.randn(topv.shape, generator=torch.Generator().manual_seed(0))
    (topv * gy.to(DEV)).sum().backward()
    h64 = t["in.x"].double().requires_grad_(True)
    W64 = {k: v.double() for k, v in W.items()}
    _, v64, _ = R.route_gemma4(h64, W64, 2, 1e-6, forced_topi=topi.cpu())
    (v64 * gy.double()).sum().backward()
    _check(h.grad.cpu(), h64.grad, "dh")


# ------------------------------------------------------------------------------------------------ experts and layer


def _layer(T=384, H=256, E=16, I=128, K=4, n_sel=3, r=8, shared=128, int4=True, act="silu", seed=0, deq=torch.float32):
    x, ol = R.make_layer(T, H, E, I, K, n_sel=n_sel, r=r, shared_inter=shared, int4=int4, seed=seed, act_name=act,
                         dtype=torch.float32, lora_b_std=0.05)
    ol.deq_dtype = deq
    return x, ol


def test_frozen_experts_fn_f32():
    """FrozenExpertsFn on fp32 rows with the reference test's counts (an empty expert), forward and dX, against the
    oracle's restatement of the reference's per-group dequant / recompute backward in fp64."""
    from smel.moe import FrozenExpertsFn
    _say("FrozenExpertsFn fp32")
    x, ol = _layer(E=6, n_sel=0, shared=None)
    counts = [9, 0, 12, 7, 15, 7]
    rows = sum(counts)
    xs = torch.randn(rows, x.shape[1])
    gy = torch.randn(rows, x.shape[1])
    W, ex, _ = to_device_layer(ol, DEV, torch.float32)
    xd = xs.to(DEV).requires_grad_(True)
    out = FrozenExpertsFn.apply(xd, counts, ex.frozen, 32, "silu")
    out.backward(gy.to(DEV))
    x64 = xs.double().requires_grad_(True)
    ref = R._FrozenExperts.apply(x64, counts, ol, torch.float64)
    ref.backward(gy.double())
    _check(out.detach().cpu(), ref.detach(), "out")
    _check(xd.grad.cpu(), x64.grad, "dx")


@pytest.mark.parametrize("case", ["int4_sel_lora", "fp32bank_sel_lora", "int4_frozen_only", "gelu_r48",
                                  "int4_bf16_dtype", "shared_split"])
def test_moe_forward_f32_against_fp64(case):
    """moe_forward on fp32 tensors (router, routed experts with selected experts and LoRA, shared expert and its
    gate): y, dX and every LoRA gradient against the fp64 oracle with the kernel's routing forced (as the
    reference's tests force HF's routing). Ranks above 32 run here (r = 48)."""
    from smel.moe import moe_forward
    _say(f"moe_forward fp32 {case}")
    kw = dict(int4=case != "fp32bank_sel_lora", n_sel=0 if case == "int4_frozen_only" else 3,
              act="gelu_tanh" if case == "gelu_r48" else "silu", r=48 if case == "gelu_r48" else 8,
              deq=torch.bfloat16 if case == "int4_bf16_dtype" else torch.float32, seed=sum(map(ord, case)) % 97)
    x, ol = _layer(**kw)
    K = 4
    gy = torch.randn(x.shape, generator=torch.Generator().manual_seed(1))
    W, ex, lora = to_device_layer(ol, DEV, torch.float32)
    if case == "shared_split":   # gate and up as separate tensors of the W dict
        assert "mlp.shared_expert.gate_proj.weight" in W
    else:                        # the stacked view LayerWeights makes
        Is = W["mlp.shared_expert.down_proj.weight"].shape[1]
        gu = torch.cat((W.pop("mlp.shared_expert.gate_proj.weight"), W.pop("mlp.shared_expert.up_proj.weight")))
        W["mlp.shared_expert.gate_up_proj.weight"] = gu
        W["mlp.shared_expert.gate_proj.weight"], W["mlp.shared_expert.up_proj.weight"] = gu[:Is], gu[Is:]
    xd = x.to(DEV).requires_grad_(True)
    seen = {}
    y = moe_forward(xd, W, ex, K, lora, stats=lambda p, v, i: seen.update(p=p, v=v, i=i.clone()))
    assert y.dtype == torch.float32 and seen["p"].dtype == torch.float32 and seen["v"].dtype == torch.float32
    y.backward(gy.to(DEV))
    torch.cuda.synchronize()
    y64, dx64, g64 = R.moe_forward_backward(x, ol, K, gy, forced_topi=seen["i"].cpu(), dtype=torch.float64)
    _check(y.detach().cpu(), y64, "y")
    _check(xd.grad.cpu(), dx64, "dx")
    if lora is not None:
        for tag, mod in (("ex", lora.experts), ("sh", lora.shared)):
            if mod is None:
                continue
            for n in LORA_NAMES:
                _check(getattr(mod, n).grad.cpu(), g64[f"{tag}_{n}"], f"d_{tag}_{n}")


def test_mlp_lora_f32_gelu_nd():
    """mlp_lora on a 3-D fp32 input (GeGLU, separate gate / up weights, LoRA r=16): y, dX and the LoRA gradients
    against the fp64 plain formula (the reference's lora_linear / lora_gate_up)."""
    from smel.lora import MLPLoRA
    from smel.moe import mlp_lora
    _say("mlp_lora fp32 GeGLU 3-D")
    torch.manual_seed(7)
    B, S, H, I, r = 3, 50, 192, 160, 16
    x = torch.randn(B, S, H)
    wg, wu, wd = torch.randn(I, H) * 0.05, torch.randn(I, H) * 0.05, torch.randn(H, I) * 0.05
    lo = MLPLoRA(H, I, r, 32.0)
    with torch.no_grad():
        for n in ("B_gate", "B_up", "B_down"):
            getattr(lo, n).normal_(0, 0.05)
    lod = MLPLoRA(H, I, r, 32.0).to(DEV)
    with torch.no_grad():
        for n in LORA_NAMES:
            getattr(lod, n).copy_(getattr(lo, n))
    xd = x.to(DEV).requires_grad_(True)
    y = mlp_lora(xd, wg.to(DEV), wu.to(DEV), wd.to(DEV), lod, act_name="gelu_tanh")
    gy = torch.randn(B, S, H)
    y.backward(gy.to(DEV))
    x64 = x.double().reshape(-1, H).requires_grad_(True)
    L64 = {n: getattr(lo, n).detach().double().requires_grad_(True) for n in LORA_NAMES}
    y64 = R.mlp_lora(x64, torch.cat((wg, wu)).double(), wd.double(), L64, lo.scale, "gelu_tanh")
    y64.backward(gy.double().reshape(-1, H))
    _check(y.detach().cpu().reshape(-1, H), y64.detach(), "y")
    _check(xd.grad.cpu().reshape(-1, H), x64.grad, "dx")
    for n in LORA_NAMES:
        _check(getattr(lod, n).grad.cpu(), L64[n].grad, f"d_{n}")


def test_c1_golden_f32(golden_c1):
    """moe_forward on the reference's own C1 inputs in fp32 (the golden outputs were written by the reference's fp32
    path): the HIP router's ids equal the golden ones, and y, dX and all twelve LoRA gradients match the golden
    values at the reference's fp32 bar."""
    from smel.moe import moe_forward
    _say("C1 golden fp32")
    t = golden_c1
    W, ex, lora = to_device_layer(c1_layer(t), DEV, torch.float32)
    x = t["in.x"].to(DEV).requires_grad_(True)
    seen = {}
    y = moe_forward(x, W, ex, 2, lora, stats=lambda p, v, i: seen.update(p=p.clone(), v=v.clone(), i=i.clone()))
    y.backward(t["in.gy"].to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(seen["i"].cpu(), t["out.topi"])
    _check(seen["p"].cpu(), t["out.probs"], "probs")
    _check(seen["v"].cpu(), t["out.topv"], "topv")
    _check(y.detach().cpu(), t["out.y"], "y")
    _check(x.grad.cpu(), t["out.dx"], "dx")
    for tag, mod in (("ex", lora.experts), ("sh", lora.shared)):
        for n in LORA_NAMES:
            _check(getattr(mod, n).grad.cpu(), t[f"out.d_{tag}_{n}"], f"d_{tag}_{n}")


def test_c1_golden_f32_frozen_only(golden_c1):
    """The golden frozen-only layer (no selected experts, no LoRA) in fp32: y and dX."""
    from smel.moe import moe_forward
    t = golden_c1
    W, ex, _ = to_device_layer(c1_layer(t, with_sel=False), DEV, torch.float32)
    x = t["in.x"].to(DEV).requires_grad_(True)
    y = moe_forward(x, W, ex, 2, None)
    y.backward(t["in.gy"].to(DEV))
    _check(y.detach().cpu(), t["out.y_frozen_only"], "y")
    _check(x.grad.cpu(), t["out.dx_frozen_only"], "dx")


def test_routed_experts_f32_bad_ids_reported():
    """fp32 routed_experts with an expert id outside [0, E): the slot is dropped (a zero row) and the error is
    reported without a host synchronisation, by check_routing_errors()."""
    from smel.moe import check_routing_errors, routed_experts
    x, ol = _layer(n_sel=0, shared=None)
    W, ex, _ = to_device_layer(ol, DEV, torch.float32)
    T = x.shape[0]
    topi = torch.randint(0, ol.E, (T, 4)).to(DEV)
    topi[3, 1] = ol.E + 2
    topv = torch.full((T, 4), 0.25, device=DEV)
    routed_experts(x.to(DEV), topv, topi, ex)
    with pytest.raises(IndexError):
        check_routing_errors()
    check_routing_errors()   # reported once


# ------------------------------------------------------------------------------------------------ bf16 beyond the bf16 kernels


@pytest.mark.parametrize("case", ["rank48", "hidden200_group8", "inter100"])
def test_bf16_layer_outside_bf16_kernel_limits(case):
    """bf16 activations of shapes the bf16 kernels do not take (LoRA rank above 32, a hidden size that is not a
    multiple of 64 with int4 groups of 8, an expert / shared intermediate size that is not a multiple of 32) run on
    the fp32 kernels with bf16 in and out: y, dX and every LoRA gradient against the fp32 oracle at the bf16 bar
    (the reference takes these shapes; its bf16 tests compare at 2e-2)."""
    from helpers import assert_close_bf16
    from smel.moe import moe_forward
    _say(f"bf16 layer beyond the bf16 kernels: {case}")
    H, I, group, r = {"rank48": (256, 128, 64, 48), "hidden200_group8": (200, 96, 8, 8),
                      "inter100": (256, 100, 4, 16)}[case]
    x, ol = R.make_layer(320, H, 16, I, 4, n_sel=3, r=r, shared_inter=I, group=group, seed=11, lora_b_std=0.05)
    W, ex, lora = to_device_layer(ol, DEV)
    gy = torch.randn(x.shape, generator=torch.Generator().manual_seed(2)).bfloat16()
    xd = x.to(DEV).requires_grad_(True)
    seen = {}
    y = moe_forward(xd, W, ex, 4, lora, stats=lambda p, v, i: seen.update(v=v, i=i.clone()))
    assert y.dtype == torch.bfloat16 and seen["v"].dtype == torch.bfloat16
    y.backward(gy.to(DEV))
    torch.cuda.synchronize()
    y32, dx32, g32 = R.moe_forward_backward(x.float(), ol, 4, gy.float(), forced_topi=seen["i"].cpu(),
                                            dtype=torch.float32)
    e, m, c = assert_close_bf16(y.detach().float().cpu(), y32, "y")
    _say(f"  y: rel {e:.2e} cos {c:.7f}")
    e, m, c = assert_close_bf16(xd.grad.float().cpu(), dx32, "dx")
    _say(f"  dx: rel {e:.2e} cos {c:.7f}")
    for tag, mod in (("ex", lora.experts), ("sh", lora.shared)):
        for n in LORA_NAMES:
            e, m, c = assert_close_bf16(getattr(mod, n).grad.float().cpu(), g32[f"{tag}_{n}"], f"d_{tag}_{n}")
            _say(f"  d_{tag}_{n}: rel {e:.2e}")


def test_bf16_frozen_experts_and_route_hidden_200():
    """FrozenExpertsFn and route() on bf16 rows whose hidden size (200) the bf16 kernels do not take: the fp32 kernels
    with bf16 in and out, against the fp32 oracle at the bf16 bar; the router's ids equal the oracle's on the same
    logits' ordering (no near-ties here)."""
    from helpers import assert_close_bf16
    from smel.moe import FrozenExpertsFn, route
    _say("bf16 FrozenExpertsFn / route, hidden 200")
    x, ol = R.make_layer(256, 200, 6, 96, 2, n_sel=0, group=8, seed=4)
    W, ex, _ = to_device_layer(ol, DEV)
    counts = [9, 0, 12, 7, 15, 7]
    xs = x[:sum(counts)].bfloat16()
    gy = torch.randn(xs.shape, generator=torch.Generator().manual_seed(3)).bfloat16()
    xd = xs.to(DEV).requires_grad_(True)
    out = FrozenExpertsFn.apply(xd, counts, ex.frozen, 32, "silu")
    assert out.dtype == torch.bfloat16
    out.backward(gy.to(DEV))
    x32 = xs.float().requires_grad_(True)
    ref = R._FrozenExperts.apply(x32, counts, ol, torch.float32)
    ref.backward(gy.float())
    assert_close_bf16(out.detach().float().cpu(), ref.detach(), "out")
    assert_close_bf16(xd.grad.float().cpu(), x32.grad, "dx")
    xr = x.bfloat16().to(DEV)
    probs, topv, topi = route(xr, W["mlp.gate.weight"], 2)
    assert topv.dtype == torch.bfloat16
    p32, _, i32 = R.route(x.bfloat16().float(), ol.gate_w.float(), 2)
    assert torch.equal(topi.cpu(), i32)
    assert_close_bf16(probs.cpu(), p32, "probs", rel=1e-5)
