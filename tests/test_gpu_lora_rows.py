"""smel_lora_rows_sum (include/smel_moe.h): the bf16 LoRA rows the LoRA gradients take, from the per-column-block fp32
partials smel_gmm_bwd_lr's down backward writes (the autograd of lora_gate_up's B products, smel/lora.py:72-83).
Against the same sum done here in fp32 in block order from 0 (the order the gate_up backward sums them in), bit for
bit; only the rows of SEL tiles (sel on) and SHARED tiles (sh on) are written, every other row keeps its sentinel."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
KIND = {"int4": 0, "bf16": 1, "sel": 2, "shared": 3}


def _tiles(groups):
    """Tile list {group, row0, row1, gk} of up to 128-row tiles over consecutive groups [(kind, rows), ...]."""
    out, r0 = [], 0
    for g, (kind, n) in enumerate(groups):
        for i in range(0, n, 128):
            out.append((g, r0 + i, r0 + min(n, i + 128), KIND[kind] << 16))
        r0 += n
    return torch.tensor(out, dtype=torch.int32), r0


@pytest.mark.parametrize("parts,planes,sel,sh", [(2, 1, 1, 1), (3, 2, 1, 0), (1, 1, 0, 1), (5, 2, 1, 1)])
def test_lora_rows_sum_bitexact(parts, planes, sel, sh):
    from smel import _lib as L
    print(f"lora_rows_sum parts{parts} planes{planes} sel{sel} sh{sh}", flush=True)
    groups = [("int4", 200), ("sel", 300), ("int4", 5), ("sel", 127), ("bf16", 64), ("shared", 257)]
    tiles, M = _tiles(groups)
    g = torch.Generator().manual_seed(parts * 10 + planes)
    part = torch.randn(M, parts, planes, 32, generator=g) * 3
    sentinel = torch.full((M, 32 * planes), -7.0).to(torch.bfloat16)
    want = sentinel.clone()
    kinds = [KIND[k] for k, _ in groups]
    for t in tiles.tolist():
        k = kinds[t[0]]
        if (k == KIND["sel"] and sel) or (k == KIND["shared"] and sh):
            v = torch.zeros(t[2] - t[1], planes, 32)
            for p in range(parts):
                v = v + part[t[1]:t[2], p]
            want[t[1]:t[2]] = v.reshape(-1, 32 * planes).to(torch.bfloat16)
    ext = sentinel.to(DEV)
    td, pd = tiles.reshape(-1).to(DEV), part.to(DEV)
    nt = torch.tensor([len(tiles)], dtype=torch.int32, device=DEV)
    L.call("smel_lora_rows_sum", L.ptr(td), L.ptr(nt), len(tiles) + 3, None, sel, sh, L.ptr(pd), parts, planes,
           L.ptr(ext), L.stream())
    torch.cuda.synchronize()
    assert torch.equal(ext.cpu().view(torch.int16), want.view(torch.int16))
