"""smel_dispatch_noalloc (the allocation-free variant of smel_dispatch, workspace in the library's own per-GPU scratch
array) against smel_dispatch with a caller workspace: bit-exact counts, offsets, permutation, inverse, tile list,
tile count and error flags, on two calls in a row, the second smaller than the first (so it reads nothing the first
left behind), and a host-side rejection of a call too large for the scratch array. Through the C-ABI."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(entry, ids, T, K, E, shared_rows, gkind):
    from smel import _lib as L
    lib = L.load()
    TK = T * K
    maxt = lib.smel_dispatch_max_tiles(TK, E, shared_rows, 128)
    i32 = lambda n, v=-7: torch.full((max(n, 1),), v, dtype=torch.int32, device=DEV)   # poisoned outputs
    out = dict(counts=i32(E), offsets=i32(E + 1), order=i32(TK), inv=i32(TK), tiles=i32(maxt * 4),
               tiles_g=i32(maxt * 4), ntiles=i32(1), err=i32(1))
    args = [L.ptr(ids), int(ids.dtype == torch.int64), T, K, E, shared_rows, 128, L.ptr(gkind)] + \
           [L.ptr(out[k]) for k in ("counts", "offsets", "order", "inv", "tiles", "tiles_g", "ntiles", "err")]
    if entry == "smel_dispatch":
        ws = torch.empty(max(1, lib.smel_dispatch_ws_size(TK, E)), dtype=torch.int32, device=DEV)
        L.call(entry, *args, 0, None, None, L.ptr(ws), L.stream())
    else:
        L.call(entry, *args, L.stream())
    torch.cuda.synchronize()
    n = int(out["ntiles"][0])
    res = {k: v.cpu().numpy() for k, v in out.items()}
    res["tiles"] = res["tiles"][:4 * n]
    res["tiles_g"] = res["tiles_g"][:4 * n]
    return res


def _ids(T, K, E, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    p = 1.0 / torch.arange(1, E + 1, dtype=torch.float64) ** 1.2          # skewed: hot experts span several tiles
    ids = torch.stack([torch.multinomial(p, K, replacement=False, generator=g) for _ in range(T)])
    return ids.to(dtype).to(DEV)


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_noalloc_dispatch_matches_workspace_dispatch(dtype):
    from smel import _lib as L
    cases = [(4092, 8, 256, 4092), (300, 4, 16, 0)]                     # second call smaller than the first
    for i, (T, K, E, sh) in enumerate(cases):
        print(f"no-alloc dispatch call {i}: T{T} K{K} E{E} shared{sh} {dtype}", flush=True)
        ids = _ids(T, K, E, 11 + i, dtype)
        gkind = torch.arange(E + (1 if sh else 0), dtype=torch.int32, device=DEV) * 3
        want = _run("smel_dispatch", ids, T, K, E, sh, gkind)
        got = _run("smel_dispatch_noalloc", ids, T, K, E, sh, gkind)
        assert want["err"][0] == 0 and got["err"][0] == 0
        for k in want:
            assert np.array_equal(got[k], want[k]), (i, k)
    lib = L.load()
    assert lib.smel_dispatch_noalloc_max_ws() == 1 << 18
    # too large for the scratch array: rejected on the host, before any launch
    big_T = 65536
    assert lib.smel_dispatch_ws_size(big_T * 8, 512) > lib.smel_dispatch_noalloc_max_ws()
    rc = lib.smel_dispatch_noalloc(1, 0, big_T, 8, 512, 0, 128, None, 1, 1, 1, 1, 1, None, 1, 1, None)
    assert rc == -2 and b"scratch" in lib.smel_last_error()
