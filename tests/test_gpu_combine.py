"""smel_combine / smel_dx_reduce (include/smel_moe.h) called through the C-ABI on their own: the weighted combine of
routed_experts (smel/moe.py:248-252, + the shared add of :263) and the dX gather-reduce (the autograd of
xs = x2d[tok], smel/moe.py:223), against the fp64 sum of the same rows (within the bf16 rounding: the kernels sum
in fp32 in a fixed order and round once). Slots dropped by the dispatch (inv < 0) have NaN rows here, so
a kernel that read them would fail; K up to 16, the shared row from Y's tail or from its own buffer, and bitwise
repeatability."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(got, exact):
    """bf16 results against the exact (fp64) sums: within the bf16 rounding (half a unit in the last place, at most
    2^-8 of the value) plus the fp32 accumulation error of a few terms of magnitude below 4."""
    err = (got.double() - exact).abs()
    return bool((err <= 2.0 ** -8 * exact.abs() + 1e-5).all())


def _rows(n, H, g):
    return (torch.randn(n, H, generator=g) * 0.5).to(torch.bfloat16)


@pytest.mark.parametrize("T,K,H,shared", [(300, 8, 2048, "tail"), (257, 12, 2816, "own"), (64, 1, 512, "none"),
                                          (33, 16, 1032, "tail")])
def test_combine_against_fp64(T, K, H, shared):
    from smel import _lib as L
    print(f"combine T{T} K{K} H{H} shared={shared}", flush=True)
    g = torch.Generator().manual_seed(T * 31 + K)
    TK = T * K
    Y = _rows(TK + (T if shared == "tail" else 0), H, g)
    topv = torch.rand(T, K, generator=g)
    inv = torch.arange(TK, dtype=torch.int32)
    drop = torch.rand(TK, generator=g) < 0.1
    inv[drop] = -1
    Y[:TK][drop] = float("nan")   # a dropped slot's row was never written
    sg = torch.rand(T, generator=g) if shared != "none" else None
    Ysh = _rows(T, H, g) if shared == "own" else None
    w = torch.where(drop.view(T, K), torch.zeros_like(topv), topv).double()
    Yk = torch.nan_to_num(Y[:TK].double(), nan=0.0).view(T, K, H)
    want = (w.unsqueeze(-1) * Yk).sum(1)
    if sg is not None:
        want += sg.double().unsqueeze(-1) * (Ysh if Ysh is not None else Y[TK:]).double()
    d = lambda x: x.to(DEV) if x is not None else None
    Yd, tv, ivd, sgd, yshd = d(Y), d(topv), d(inv), d(sg), d(Ysh)
    outs = []
    for _ in range(2):
        out = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=DEV)
        L.call("smel_combine", L.ptr(Yd), L.ptr(tv), L.ptr(ivd), L.ptr(sgd), L.ptr(yshd), T, K, H, L.ptr(out),
               L.stream())
        torch.cuda.synchronize()
        outs.append(out.cpu())
    assert torch.isfinite(outs[0].float()).all()
    assert _close(outs[0], want)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


@pytest.mark.parametrize("T,K,H,shared,router", [(300, 8, 2048, "tail", True), (129, 12, 2816, "own", False),
                                                 (40, 16, 520, "none", True), (17, 2, 64, "tail", False)])
def test_dx_reduce_against_fp64(T, K, H, shared, router):
    from smel import _lib as L
    print(f"dx_reduce T{T} K{K} H{H} shared={shared} router={router}", flush=True)
    g = torch.Generator().manual_seed(T * 7 + K)
    TK = T * K
    dxs = _rows(TK + (T if shared == "tail" else 0), H, g)
    inv = torch.arange(TK, dtype=torch.int32)
    drop = torch.rand(TK, generator=g) < 0.1
    inv[drop] = -1
    dxs[:TK][drop] = float("nan")
    dxsh = _rows(T, H, g) if shared == "own" else None
    dxr = _rows(T, H, g) if router else None
    want = torch.nan_to_num(dxs[:TK].double(), nan=0.0).view(T, K, H).sum(1)
    if shared != "none":
        want += (dxsh if dxsh is not None else dxs[TK:]).double()
    if dxr is not None:
        want += dxr.double()
    d = lambda x: x.to(DEV) if x is not None else None
    dd, dr, ivd, dsh = d(dxs), d(dxr), d(inv), d(dxsh)
    outs = []
    for _ in range(2):
        out = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=DEV)
        L.call("smel_dx_reduce", L.ptr(dd), L.ptr(dr), L.ptr(ivd), int(shared != "none"), L.ptr(dsh), T, K, H,
               L.ptr(out), L.stream())
        torch.cuda.synchronize()
        outs.append(out.cpu())
    assert torch.isfinite(outs[0].float()).all()
    assert _close(outs[0], want)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


def test_combine_rejects_more_than_16_slots():
    from smel import _lib as L
    assert L.load().smel_combine(None, None, None, None, None, 4, 17, 64, None, None) != 0
    assert L.load().smel_dx_reduce(None, None, None, 0, None, 4, 17, 64, None, None) != 0
