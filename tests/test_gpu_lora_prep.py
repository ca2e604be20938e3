"""smel_lora_prep / smel_lora_prep_sets (include/smel_moe.h): every bf16 layout of the LoRA factors against a torch
construction of its definition (the layouts the K-extensions and the LoRA projections read, built from the fp32
factors of smel/lora.py:17-58), bit for bit, for one and two planes, ranks up to 32, sizes that end inside a
128-wide chunk, and two sets in one launch. Outputs start as NaN, so an element the kernel leaves unwritten fails.
Dimensions that are not multiples of 32 (which no GEMM of the layer takes) are refused on the host."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = ("fwd_gu", "fwd_dn", "a_gu", "a_dn", "bt_dn", "bt_gu", "at_gu", "at_dn")


def _factors(n, r, Hd, In, seed):
    g = torch.Generator().manual_seed(seed)
    f = lambda *s: torch.randn(*s, generator=g) * 0.3
    return dict(A_gate=f(n, r, Hd), B_gate=f(n, In, r), A_up=f(n, r, Hd), B_up=f(n, In, r), A_down=f(n, r, In),
                B_down=f(n, Hd, r))


def _expected(F, r, P, Hd, In):
    """The layouts from their definitions: 32 rank slots per plane; with one plane the gate ranks sit in slots
    0..r-1 and the up ranks in 16..16+r-1, with two planes each projection has its own plane (slots 0..r-1)."""
    n = F["A_gate"].shape[0]

    def gate_rank(plane, j):
        return j if plane == 0 and j < r else -1

    def up_rank(plane, j):
        if P == 1:
            return j - 16 if 16 <= j < 16 + r else -1
        return j if plane == 1 and j < r else -1

    z = lambda *s: torch.zeros(*s)
    fwd_gu, fwd_dn, a_gu, a_dn = z(n, 2 * In, 32), z(n, Hd, 32), z(P, n, 32, Hd), z(n, 32, In)
    bt_dn, bt_gu = z(n, 32, Hd), z(P, n, 32, 2 * In)
    fwd_gu[:, :In, :r] = F["B_gate"]
    fwd_dn[:, :, :r] = F["B_down"]
    a_dn[:, :r, :] = F["A_down"]
    bt_dn[:, :r, :] = F["B_down"].transpose(1, 2)
    for j in range(32):
        k = up_rank(P - 1, j)
        if k >= 0:
            fwd_gu[:, In:, j] = F["B_up"][:, :, k]
        for pl in range(P):
            kg, ku = gate_rank(pl, j), up_rank(pl, j)
            if kg >= 0:
                a_gu[pl, :, j, :] = F["A_gate"][:, kg, :]
                bt_gu[pl, :, j, :In] = F["B_gate"][:, :, kg]
            if ku >= 0:
                a_gu[pl, :, j, :] = F["A_up"][:, ku, :]
                bt_gu[pl, :, j, In:] = F["B_up"][:, :, ku]
    out = dict(fwd_gu=fwd_gu, fwd_dn=fwd_dn, a_gu=a_gu, a_dn=a_dn, bt_dn=bt_dn, bt_gu=bt_gu,
               at_gu=a_gu.permute(1, 0, 3, 2), at_dn=a_dn.transpose(1, 2))
    return {k: v.contiguous().to(torch.bfloat16) for k, v in out.items()}


def _outputs(n, P, Hd, In):
    shapes = dict(fwd_gu=(n, 2 * In, 32), fwd_dn=(n, Hd, 32), a_gu=(P, n, 32, Hd), a_dn=(n, 32, In),
                  bt_dn=(n, 32, Hd), bt_gu=(P, n, 32, 2 * In), at_gu=(n, P, Hd, 32), at_dn=(n, In, 32))
    return {k: torch.full(s, float("nan"), dtype=torch.bfloat16, device=DEV) for k, s in shapes.items()}


def _set(L, F, out, n, r):
    dev = {k: v.to(DEV).contiguous() for k, v in F.items()}
    s = L.LoraSet(*[L.ptr(dev[k]) for k in ("A_gate", "B_gate", "A_up", "B_up", "A_down", "B_down")], n, r)
    for k in NAMES:
        setattr(s, k, L.ptr(out[k]))
    return s, dev


def _check(out, want, tag):
    for k in NAMES:
        got = out[k].cpu()
        assert got.shape == want[k].shape, (tag, k)
        assert torch.equal(got.view(torch.int16), want[k].view(torch.int16)), (tag, k)


@pytest.mark.parametrize("n,r,P,Hd,In", [(3, 4, 1, 256, 128), (2, 16, 1, 384, 320), (2, 24, 2, 256, 704),
                                         (1, 32, 2, 192, 96), (12, 16, 1, 2048, 512)])
def test_lora_prep_layouts(n, r, P, Hd, In):
    from smel import _lib as L
    print(f"lora_prep n{n} r{r} planes{P} Hd{Hd} In{In}", flush=True)
    F = _factors(n, r, Hd, In, n * 100 + r)
    out = _outputs(n, P, Hd, In)
    s, keep = _set(L, F, out, n, r)
    L.call("smel_lora_prep_sets", ctypes.byref(s), 1, P, Hd, In, L.stream())
    torch.cuda.synchronize()
    _check(out, _expected(F, r, P, Hd, In), "one set")


def test_lora_prep_two_sets_one_launch():
    from smel import _lib as L
    print("lora_prep two sets", flush=True)
    Hd, In, P = 320, 192, 2
    sets, keep, outs, Fs = [], [], [], []
    for i, (n, r) in enumerate([(5, 20), (1, 8)]):
        F = _factors(n, r, Hd, In, 7 + i)
        out = _outputs(n, P, Hd, In)
        s, dev = _set(L, F, out, n, r)
        sets.append(s)
        keep.append(dev)
        outs.append(out)
        Fs.append((F, r))
    arr = (L.LoraSet * 2)(*sets)
    L.call("smel_lora_prep_sets", arr, 2, P, Hd, In, L.stream())
    torch.cuda.synchronize()
    for i, (F, r) in enumerate(Fs):
        _check(outs[i], _expected(F, r, P, Hd, In), f"set {i}")


def test_lora_prep_rejects_unaligned_dimensions():
    from smel import _lib as L
    F = _factors(1, 4, 64, 48, 1)
    out = _outputs(1, 1, 64, 48)
    s, keep = _set(L, F, out, 1, 4)
    assert L.load().smel_lora_prep_sets(ctypes.byref(s), 1, 1, 64, 48, None) == -2   # In = 48: not a multiple of 32
