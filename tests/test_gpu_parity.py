"""HIP kernels vs the CPU oracle, through the C-ABI (via the drop-in smel.* API or direct entry points).

Bars: bit-exact for integer / byte / index results (dequantized values, top-k ids given identical logits, dispatch
permutation, counts, offsets, tile list); bf16 outputs and gradients within ||d||/||ref|| <= 2e-2,
max|d| <= 2e-2 max|ref| and cosine >= 0.9999 against the fp32 oracle on the same inputs (and the same routing, which
the tests force as the reference's own tests do, tests/helpers.py:89-106); bitwise run-to-run determinism.
"""
import ctypes

import numpy as np
import pytest
import torch

from helpers import LORA_NAMES, QUANT_CASES, assert_close_bf16, to_device_layer
from oracle import intref
from oracle import moe_ref as R

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _u16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _lib():
    from smel import _lib
    return _lib


def _say(msg):
    print(msg, flush=True)


# ------------------------------------------------------------------------------------------------------- dequant


@pytest.mark.parametrize("case", QUANT_CASES)
def test_dequant_golden_bitexact(golden_quant, case):
    from smel.quant import dequant_int4
    _say(f"dequant golden {case}")
    g = golden_quant
    q, s, z = (g[f"quant.{case}.{k}"].to(DEV) for k in ("q", "scale", "zero"))
    out = dequant_int4(q, s, z, torch.bfloat16)
    want = intref.dequant_bits(g[f"quant.{case}.q"].numpy(), _u16(g[f"quant.{case}.scale"]),
                               _u16(g[f"quant.{case}.zero"]))
    assert np.array_equal(_u16(out), want)
    f32 = dequant_int4(q, s, z, torch.float32)
    assert torch.equal(f32.cpu(), g[f"quant.{case}.deq_f32"])


@pytest.mark.parametrize("shape,group", [((256, 1024, 2048), 64), ((7, 64, 32), 32), ((3, 5, 96), 32),
                                         ((2, 3, 6), 2)])
def test_dequant_random_bitexact(shape, group):
    from smel.quant import dequant_int4
    _say(f"dequant random {shape} g{group}")
    gen = torch.Generator().manual_seed(sum(shape))
    E, N, K = shape
    q = torch.randint(0, 256, (E, N, K // 2), generator=gen, dtype=torch.uint8)
    s = (torch.rand(E, N, K // group, generator=gen) * 0.01 + 1e-4).to(torch.bfloat16)
    z = (torch.randn(E, N, K // group, generator=gen) * 0.05).to(torch.bfloat16)
    out = dequant_int4(q.to(DEV), s.to(DEV), z.to(DEV))
    assert np.array_equal(_u16(out), intref.dequant_bits(q.numpy(), _u16(s), _u16(z)))


# ------------------------------------------------------------------------------------------------------- packing
# The GEMMs read weights in the fragment layout of include/smel_moe.h (SMEL_PACK_*); these tests invert that layout
# with numpy index arithmetic and require the round trip to be the identity, with zeros in the padding.


def _unpack_q4(qf, szf, rows, K):
    nf, nk = -(-rows // 32), -(-K // 64)
    nk4 = -(-nk // 4)
    q = qf.reshape(nf, nk, 2, 32, 16).transpose(0, 3, 1, 2, 4).reshape(nf * 32, nk * 32)
    sz = szf.reshape(nf, nk4, 2, 32, 4).transpose(0, 3, 1, 4, 2).reshape(nf * 32, nk4 * 4, 2)
    return q, sz


@pytest.mark.parametrize("E,R,K,group", [(3, 64, 192, 64), (2, 32, 96, 32), (1, 96, 2048, 64)])
def test_pack_int4_roundtrip(E, R, K, group):
    L = _lib()
    _say(f"pack int4 E{E} R{R} K{K} g{group}")
    gen = torch.Generator().manual_seed(E * R + K)
    q = torch.randint(0, 256, (E, R, K // 2), generator=gen, dtype=torch.uint8)
    sc = torch.randint(0, 65536, (E, R, K // group), generator=gen, dtype=torch.int32).to(torch.int16)
    ze = torch.randint(0, 65536, (E, R, K // group), generator=gen, dtype=torch.int32).to(torch.int16)
    lib = L.load()
    rows = E * R
    qf = torch.empty(lib.smel_packed_bytes(L.PACK_Q4, rows, K), dtype=torch.uint8, device=DEV)
    szf = torch.empty(lib.smel_packed_bytes(L.PACK_SZ, rows, K) // 4, dtype=torch.int32, device=DEV)
    qd, sd, zd = q.to(DEV), sc.to(DEV), ze.to(DEV)
    L.call("smel_pack_int4", L.ptr(qd), L.ptr(sd), L.ptr(zd), rows, K, group, L.ptr(qf), L.ptr(szf), L.stream())
    uq, usz = _unpack_q4(qf.cpu().numpy(), szf.cpu().numpy().view(np.uint32), rows, K)
    qn = q.reshape(rows, K // 2).numpy()
    assert np.array_equal(uq[:, :K // 2], qn)
    assert not uq[:, K // 2:].any()
    s16 = sc.reshape(rows, -1).numpy().view(np.uint16).astype(np.uint32)
    z16 = ze.reshape(rows, -1).numpy().view(np.uint16).astype(np.uint32)
    nks = usz.shape[1]
    col = 64 * np.arange(nks)[:, None] + 32 * np.arange(2)[None, :]          # [ks][h]
    inside = col < K
    g = np.minimum(col, K - 1) // group
    want = np.where(inside[None], s16[:, g] | (z16[:, g] << 16), 0).astype(np.uint32)
    assert np.array_equal(usz, want)


@pytest.mark.parametrize("rows,K,ld", [(33, 72, 80), (64, 2048, 2048), (32, 32, 32)])
def test_pack_bf16_roundtrip(rows, K, ld):
    L = _lib()
    _say(f"pack bf16 rows{rows} K{K} ld{ld}")
    gen = torch.Generator().manual_seed(rows + K)
    w = torch.randn(rows, ld, generator=gen).to(torch.bfloat16)
    lib = L.load()
    wf = torch.empty(lib.smel_packed_bytes(L.PACK_BF16, rows, K) // 2, dtype=torch.bfloat16, device=DEV)
    wd = w.to(DEV)
    L.call("smel_pack_bf16", L.ptr(wd), rows, K, ld, L.ptr(wf), L.stream())
    nf, nk = -(-rows // 32), -(-K // 64)
    u = _u16(wf).reshape(nf, nk, 4, 2, 32, 8).transpose(0, 4, 1, 3, 2, 5).reshape(nf * 32, nk * 64)
    assert np.array_equal(u[:rows, :K], _u16(w)[:, :K])
    assert not u[rows:].any() and not u[:, K:].any()


# The backward GEMM's transposed layouts (SMEL_PACK_* of smel_pack_int4_t / smel_pack_bf16_t), inverted the same way.


def _t_index(E, R, C):
    """(row, col) of every packed element of the transposed q / bf16 layouts, in packed order
    [e][p][ks][kq][i][fr][s][t] (bf16: [e][p][ks][fr][s][kq][i][t])."""
    nks = -(-R // 64)
    p, ks, kq, i, fr, s, t = np.meshgrid(np.arange(C // 32), np.arange(nks), np.arange(4), np.arange(16),
                                         np.arange(2), np.arange(2), np.arange(8), indexing="ij")
    return 64 * ks + 32 * s + 8 * kq + t, 32 * p + 16 * fr + i


def _realistic_sz(gen, shape):
    """Scale / zero as the reference's quantizer makes them (zero = group minimum, scale = range / 15) in bf16."""
    s = (torch.rand(*shape, generator=gen) * 0.004 + 1e-4).to(torch.bfloat16)
    z = (-7.5 * s.float() * (0.6 + 0.8 * torch.rand(*shape, generator=gen))).to(torch.bfloat16)
    return s, z


@pytest.mark.parametrize("E,R,C,group,fast", [(3, 128, 192, 64, 0), (2, 96, 64, 32, 0), (1, 1024, 2048, 64, 0),
                                              (2, 128, 256, 64, 1), (2, 64, 96, 32, 1)])
def test_pack_int4_t_roundtrip(E, R, C, group, fast):
    L = _lib()
    _say(f"pack int4 transposed E{E} R{R} C{C} g{group} fast{fast}")
    gen = torch.Generator().manual_seed(E * R + C + 1)
    q = torch.randint(0, 256, (E, R, C // 2), generator=gen, dtype=torch.uint8)
    if fast:
        sc, ze = (t.view(torch.int16) for t in _realistic_sz(gen, (E, R, C // group)))
    else:   # any bit patterns: the pairs are bf16 -> fp32 copies
        sc = torch.randint(0, 65536, (E, R, C // group), generator=gen, dtype=torch.int32).to(torch.int16)
        ze = torch.randint(0, 65536, (E, R, C // group), generator=gen, dtype=torch.int32).to(torch.int16)
    lib = L.load()
    qt = torch.empty(lib.smel_packed_t_bytes(L.PACK_Q4, E, R, C, group), dtype=torch.uint8, device=DEV)
    szt = torch.empty(lib.smel_packed_t_bytes(L.PACK_SZ, E, R, C, group) // 4, dtype=torch.int32, device=DEV)
    qd, sd, zd = q.to(DEV), sc.to(DEV), ze.to(DEV)
    L.call("smel_pack_int4_t", L.ptr(qd), L.ptr(sd), L.ptr(zd), E, R, C, group, fast, L.ptr(qt), L.ptr(szt),
           L.stream())
    nks = -(-R // 64)
    # dense nibbles of the source: low nibble = even column
    qn = q.numpy()
    dense = np.stack((qn & 15, qn >> 4), axis=-1).reshape(E, R, C)
    words = qt.cpu().numpy().view(np.uint32).reshape(E, C // 32, nks, 4, 16, 2, 2)   # [e][p][ks][kq][i][fr][s]
    nib = (words[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 15              # [..., t]
    row, col = _t_index(E, R, C)
    ok = row < R
    for e in range(E):
        got = nib[e]
        assert np.array_equal(got[ok], dense[e][row[ok], col[ok]])
        assert not got[~ok].any()
    s32 = sc.numpy().view(np.uint16).astype(np.uint32) << 16
    z32 = ze.numpy().view(np.uint16).astype(np.uint32) << 16
    pw = szt.cpu().numpy().view(np.uint32).reshape(E, C // group, nks, 4, 2, 8, 2)    # [e][g][ks][kq][s][t][pair]
    ks, kq, ss, t = np.meshgrid(np.arange(nks), np.arange(4), np.arange(2), np.arange(8), indexing="ij")
    r = 64 * ks + 32 * ss + 8 * kq + t
    rc = np.minimum(r, R - 1)
    for e in range(E):
        for g in range(C // group):
            if fast:   # even rows (s, z - 1024 s), odd rows (s / 16, z - 64 s): exact in double, rounded once
                sv = s32[e][rc, g].view(np.float32).astype(np.float64)
                zv = z32[e][rc, g].view(np.float32).astype(np.float64)
                sv, zv = np.where(t % 2 == 1, sv / 16.0, sv), np.where(t % 2 == 1, zv - 64.0 * sv, zv - 1024.0 * sv)
                sb, zb = sv.astype(np.float32).view(np.uint32), zv.astype(np.float32).view(np.uint32)
            else:      # bit copies (any pattern, NaN payloads included)
                sb, zb = s32[e][rc, g], z32[e][rc, g]
            want_s = np.where(r < R, sb, 0).astype(np.uint32)
            want_z = np.where(r < R, zb, 0).astype(np.uint32)
            assert np.array_equal(pw[e, g, ..., 0], want_s)
            assert np.array_equal(pw[e, g, ..., 1], want_z)


def test_int4_fast_ok():
    """The exactness check of the fast dequant form: reference-style groups pass; a zero far below the scale, a
    zero far above it and a scale whose 1024 multiple overflows each fail it."""
    L = _lib()
    gen = torch.Generator().manual_seed(11)
    s, z = _realistic_sz(gen, (64, 32))
    ok = torch.zeros(1, dtype=torch.int32, device=DEV)

    def check(s_, z_):
        sd, zd = s_.to(DEV), z_.to(DEV)   # kept alive until the kernel has read them
        L.call("smel_int4_fast_ok", L.ptr(sd), L.ptr(zd), s_.numel(), L.ptr(ok), L.stream())
        return int(ok.item())

    assert check(s, z) == 1
    assert check(s, torch.zeros_like(z)) == 1                         # zero = 0: z - 1024 s is -1024 s, exact
    for s_val, z_val in ((1e-3, 2.0 ** -60), (1e-8, 2.0 ** 20), (2.0 ** 120, 1.0)):
        s2, z2 = s.clone(), z.clone()
        s2[5, 7], z2[5, 7] = s_val, z_val
        assert check(s2, z2) == 0, (s_val, z_val)


@pytest.mark.parametrize("group,fast", [(64, True), (64, False), (32, True), (32, False)])
def test_gemm_dequant_bitexact(group, fast):
    """The grouped GEMMs' in-loop dequant reproduces the reference's bf16 weights bit for bit: with identity blocks
    as A, the forward GEMM returns W^T and the backward GEMM W of every expert exactly (one nonzero product per
    output, rounded to bf16 from an exact bf16 value). Both the fast dequant form and the plain one, for 64- and
    32-wide groups."""
    from smel.moe import Int4Experts, _bank_gkind, _bank_wset, _count_tiles
    L = _lib()
    _say(f"gemm dequant bit-exact g{group} fast{fast}")
    E, R, C = 3, 128, 256
    gen = torch.Generator().manual_seed(group + fast)
    q = torch.randint(0, 256, (E, R, C // 2), generator=gen, dtype=torch.uint8)
    s, z = _realistic_sz(gen, (E, R, C // group))
    if not fast:
        z[1, 3, 0] = 2.0 ** -60   # one group outside the fast form's exactness condition
    d = {"q": q.to(DEV), "scale": s.to(DEV), "zero": z.to(DEV)}
    bank = Int4Experts(d, d)
    assert bank.fast_dq("gu") == fast
    want = intref.dequant_bits(q.numpy(), _u16(s), _u16(z)).reshape(E, R, C)
    gk = _bank_gkind(bank, DEV)
    # forward: rows e*C + k carry e_k -> out[e*C + k][n] = W_e[n][k]
    w = _bank_wset(bank, "gu")
    A = torch.eye(C, dtype=torch.bfloat16).repeat(E, 1).to(DEV)
    order = torch.arange(E * C, dtype=torch.int32, device=DEV)
    tiles, nt, maxt = _count_tiles([C] * E, DEV)
    out = torch.empty(E * C, R, dtype=torch.bfloat16, device=DEV)
    L.call("smel_gmm_fwd", ctypes.byref(w), L.ptr(gk), L.ptr(tiles), L.ptr(nt), maxt, L.ptr(A), C, E * C, 0,
           L.ptr(order), E * C, 1, None, 0, 0, L.ptr(out), R, None, L.stream())
    got = _u16(out).reshape(E, C, R)
    assert np.array_equal(got, want.transpose(0, 2, 1))
    # backward (transposed layout): rows e*R + r carry e_r -> out[e*R + r][n] = W_e[r][n]
    wt = _bank_wset(bank, "gu", t=True)
    At = torch.eye(R, dtype=torch.bfloat16).repeat(E, 1).to(DEV)
    order_t = torch.arange(E * R, dtype=torch.int32, device=DEV)
    tiles, nt, maxt = _count_tiles([R] * E, DEV)
    out_t = torch.empty(E * R, C, dtype=torch.bfloat16, device=DEV)
    L.call("smel_gmm_bwd", ctypes.byref(wt), L.ptr(gk), L.ptr(tiles), L.ptr(nt), maxt, L.ptr(At), R, E * R, 0,
           L.ptr(order_t), E * R, 1, None, 0, 0, None, None, None, L.ptr(out_t), C, None, L.stream())
    assert np.array_equal(_u16(out_t).reshape(E, R, C), want)


@pytest.mark.parametrize("E,R,C", [(2, 96, 64), (1, 288, 2048), (12, 512, 2048)])
def test_pack_bf16_t_roundtrip(E, R, C):
    L = _lib()
    _say(f"pack bf16 transposed E{E} R{R} C{C}")
    gen = torch.Generator().manual_seed(E + R + C)
    w = torch.randn(E, R, C, generator=gen).to(torch.bfloat16)
    lib = L.load()
    wt = torch.empty(lib.smel_packed_t_bytes(L.PACK_BF16, E, R, C, 0) // 2, dtype=torch.bfloat16, device=DEV)
    wd = w.to(DEV)
    L.call("smel_pack_bf16_t", L.ptr(wd), E, R, C, C, L.ptr(wt), L.stream())
    nks = -(-R // 64)
    u = _u16(wt).reshape(E, C // 32, nks, 2, 2, 4, 16, 8)                            # [e][p][ks][fr][s][kq][i][t]
    u = u.transpose(0, 1, 2, 5, 6, 3, 4, 7)                                           # -> [e][p][ks][kq][i][fr][s][t]
    row, col = _t_index(E, R, C)
    ok = row < R
    src = _u16(w)
    for e in range(E):
        assert np.array_equal(u[e][ok], src[e][row[ok], col[ok]])
        assert not u[e][~ok].any()


# -------------------------------------------------------------------------------------------------------- router


def _route_logits(logits, K):
    L = _lib()
    T, E = logits.shape
    probs = torch.empty(T, E, dtype=torch.float32, device=DEV)
    topv = torch.empty(T, K, dtype=torch.bfloat16, device=DEV)
    topi = torch.empty(T, K, dtype=torch.int64, device=DEV)
    topi32 = torch.empty(T, K, dtype=torch.int32, device=DEV)
    L.call("smel_route_logits", L.ptr(logits), T, E, K, L.ptr(probs), L.ptr(topv), L.ptr(topi), L.ptr(topi32),
           L.stream())
    return probs, topv, topi, topi32


@pytest.mark.parametrize("T,E,K", [(4092, 256, 8), (128, 8, 2), (513, 128, 8), (1, 64, 1), (33, 256, 16),
                                   (700, 512, 8), (50, 257, 16)])
def test_route_ids_bitexact_given_logits(T, E, K):
    _say(f"route_logits T{T} E{E} K{K}")
    gen = torch.Generator().manual_seed(T + E)
    logits = (torch.randn(T, E, generator=gen) * 0.9).to(torch.bfloat16)
    # plant exact ties (including at the k-th place) in a third of the rows
    for t in range(0, T, 3):
        j = torch.randperm(E, generator=gen)[:4]
        logits[t, j[1:]] = logits[t, j[0]].item()
    probs, topv, topi, topi32 = _route_logits(logits.to(DEV), K)
    want_v, want_i = intref.topk(logits.float().numpy(), K)     # the id rule on identical logits
    assert np.array_equal(topi.cpu().numpy(), want_i)
    assert np.array_equal(topi32.cpu().numpy(), want_i)
    pr, tv, ti = R.route(None, None, K, logits=logits.float())
    assert np.array_equal(ti.numpy(), want_i)                  # the oracle router picks the same ids
    assert torch.allclose(probs.cpu(), pr, rtol=1e-5, atol=1e-7)
    assert torch.allclose(topv.float().cpu(), tv.float(), rtol=8e-3, atol=1e-6)


@pytest.mark.parametrize("T,H,E,K,shared", [(4092, 2048, 256, 8, True), (128, 64, 8, 2, True),
                                            (300, 256, 16, 4, False), (7, 128, 100, 3, True),
                                            (500, 256, 512, 8, True), (64, 128, 300, 16, False)])
def test_route_fused(T, H, E, K, shared):
    """Fused logits GEMM + selection: ids agree with the oracle except at bf16 near-ties of the logits, whose rate is
    reported; probs / topv / shared gate within tolerance."""
    L = _lib()
    _say(f"route fused T{T} H{H} E{E} K{K}")
    gen = torch.Generator().manual_seed(E)
    x = torch.randn(T, H, generator=gen).to(torch.bfloat16)
    gw = (torch.randn(E, H, generator=gen) * 0.02).to(torch.bfloat16)
    sg = (torch.randn(H, generator=gen) * 0.02).to(torch.bfloat16)
    probs = torch.empty(T, E, dtype=torch.float32, device=DEV)
    topv = torch.empty(T, K, dtype=torch.bfloat16, device=DEV)
    topv32 = torch.empty(T, K, dtype=torch.float32, device=DEV)
    topi = torch.empty(T, K, dtype=torch.int64, device=DEV)
    topi32 = torch.empty(T, K, dtype=torch.int32, device=DEV)
    sgate = torch.empty(T, dtype=torch.float32, device=DEV)
    xd, gwd, sgd = x.to(DEV), gw.to(DEV), sg.to(DEV)
    ldl = L.load().smel_route_ld(E, int(shared))
    lgw = torch.full((T, ldl), float("nan"), dtype=torch.bfloat16, device=DEV)
    L.call("smel_route", L.ptr(xd), L.ptr(gwd), L.ptr(sgd) if shared else None, T, H, E, K, L.ptr(probs),
           L.ptr(topv), L.ptr(topv32), L.ptr(topi), L.ptr(topi32), L.ptr(sgate) if shared else None, L.ptr(lgw),
           L.stream())
    assert torch.equal(topv32.cpu(), topv.float().cpu())       # the fp32 copy is the bf16 value itself
    logits = (x.double() @ gw.double().t())                   # exact dot products of the bf16 inputs
    lb = logits.float().to(torch.bfloat16).float()
    # the workspace holds the kernel's bf16 logits: close to the exact ones, and the selection on them is exact
    glog = lgw.float().cpu()
    assert torch.allclose(glog[:, :E].double(), logits, rtol=1e-2, atol=2e-3)
    _, sel_i = intref.topk(glog[:, :E].numpy(), K)
    assert np.array_equal(topi.cpu().numpy(), sel_i)
    assert torch.equal(topi32.cpu().long(), topi.cpu())
    if shared:
        e32 = (E + 31) // 32 * 32
        assert torch.allclose(glog[:, e32].double(), x.double() @ sg.double(), rtol=1e-2, atol=2e-3)
    _, want_i = intref.topk(lb.numpy(), K)
    got = topi.cpu().numpy()
    bad = np.where((got != want_i).any(1))[0]
    srt = np.sort(logits.numpy(), axis=1)[:, ::-1]
    for t in bad:   # a flip is only allowed where the k-th and (k+1)-th logits are within bf16 rounding
        gap = srt[t, K - 1] - srt[t, K] if K < E else np.inf
        assert gap <= 2 ** -7 * max(1.0, abs(srt[t, K - 1])), (t, gap)
    _say(f"  id flips at near-ties: {len(bad)}/{T}")
    assert len(bad) <= max(2, T // 100)
    pr = torch.softmax(lb, -1)
    assert torch.allclose(probs.cpu(), pr, rtol=2e-2, atol=1e-4)
    if shared:
        ref = torch.sigmoid((x.double() @ sg.double()).float().to(torch.bfloat16).float())
        assert torch.allclose(sgate.cpu(), ref, rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("T,H,E,K,shared", [(4092, 2048, 256, 8, True), (77, 128, 16, 3, False),
                                           (1300, 256, 512, 8, True)])
def test_route_counted_then_dispatch_counted(T, H, E, K, shared):
    """smel_route_counted + smel_dispatch_counted (the router counting the dispatch's histograms) against smel_route +
    smel_dispatch: every output bit for bit, with the workspace starting as garbage."""
    L = _lib()
    lib = L.load()
    _say(f"route/dispatch counted T{T} H{H} E{E} K{K}")
    gen = torch.Generator().manual_seed(T + E)
    xd = torch.randn(T, H, generator=gen).to(torch.bfloat16).to(DEV)
    gwd = (torch.randn(E, H, generator=gen) * 0.02).to(torch.bfloat16).to(DEV)
    sgd = (torch.randn(H, generator=gen) * 0.02).to(torch.bfloat16).to(DEV) if shared else None
    TK, sh = T * K, (T if shared else 0)
    maxt = lib.smel_dispatch_max_tiles(TK, E, sh, 128)
    gk = torch.arange(E + (1 if shared else 0), dtype=torch.int32, device=DEV) * 5

    def run(counted):
        f32 = lambda *s: torch.full(s, float("nan"), dtype=torch.float32, device=DEV)
        i32 = lambda n: torch.full((n,), -7, dtype=torch.int32, device=DEV)
        o = dict(probs=f32(T, E), topv=torch.zeros(T, K, dtype=torch.bfloat16, device=DEV), topv32=f32(T, K),
                 topi=torch.zeros(T, K, dtype=torch.int64, device=DEV), topi32=i32(TK), sgate=f32(T),
                 lg=torch.zeros(T, lib.smel_route_ld(E, int(shared)), dtype=torch.bfloat16, device=DEV),
                 counts=i32(E), offsets=i32(E + 1), order=i32(TK), inv=i32(TK), tiles=i32(4 * maxt),
                 tiles_g=i32(4 * maxt), ntiles=i32(1), err=i32(1), tiles_m=i32(4 * maxt), ntiles_m=i32(1))
        ws = torch.randint(-1000, 1000, (max(1, lib.smel_dispatch_ws_size(TK, E)),), dtype=torch.int32, device=DEV)
        route = [L.ptr(xd), L.ptr(gwd), L.ptr(sgd), T, H, E, K] + [L.ptr(o[k]) for k in
                                                                   ("probs", "topv", "topv32", "topi", "topi32")] + \
                [L.ptr(o["sgate"]) if shared else None, L.ptr(o["lg"])]
        if counted:
            L.call("smel_route_counted", *route, L.ptr(ws), L.stream())
        else:
            L.call("smel_route", *route, L.stream())
        L.call("smel_dispatch_counted" if counted else "smel_dispatch", L.ptr(o["topi32"]), 0, T, K, E, sh, 128,
               L.ptr(gk), *[L.ptr(o[k]) for k in ("counts", "offsets", "order", "inv", "tiles", "tiles_g", "ntiles",
                                                  "err")], 160, L.ptr(o["tiles_m"]), L.ptr(o["ntiles_m"]), L.ptr(ws),
               L.stream())
        torch.cuda.synchronize()
        return {k: v.cpu() for k, v in o.items()}

    want, got = run(False), run(True)
    assert want["err"][0] == 0
    for k in want:
        if k == "sgate" and not shared:
            continue
        a, b = want[k], got[k]
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                           b.view(torch.int16) if b.dtype == torch.bfloat16 else b) or \
            (a.dtype.is_floating_point and torch.equal(torch.nan_to_num(a, 7.0), torch.nan_to_num(b, 7.0))), k


# ------------------------------------------------------------------------------------------------------ dispatch


def _dispatch(ids, T, K, E, shared_rows=0, m_tile=128, gkind=None, merge_rows=0):
    L = _lib()
    TK = T * K
    maxt = L.load().smel_dispatch_max_tiles(TK, E, shared_rows, m_tile)
    i32 = lambda n: torch.full((n,), -7, dtype=torch.int32, device=DEV)
    counts, offsets, order, inv = i32(E), i32(E + 1), i32(max(TK, 1)), i32(max(TK, 1))
    tiles, tiles_g, ntiles, err = i32(maxt * 4), i32(maxt * 4), i32(1), i32(1)
    tiles_m, ntiles_m = i32(maxt * 4), i32(1)
    ws = i32(max(1, L.load().smel_dispatch_ws_size(TK, E)))   # garbage-filled: the kernels must not rely on zeros
    gk = torch.tensor(gkind, dtype=torch.int32, device=DEV) if gkind is not None else None
    L.call("smel_dispatch", L.ptr(ids), int(ids.dtype == torch.int64), T, K, E, shared_rows, m_tile, L.ptr(gk),
           L.ptr(counts), L.ptr(offsets), L.ptr(order), L.ptr(inv), L.ptr(tiles), L.ptr(tiles_g), L.ptr(ntiles),
           L.ptr(err), merge_rows, L.ptr(tiles_m) if merge_rows else None, L.ptr(ntiles_m) if merge_rows else None,
           L.ptr(ws), L.stream())
    out = [a.cpu().numpy() for a in (counts, offsets, order, inv, tiles, ntiles, err)]
    _dispatch.grouped = tiles_g.cpu().numpy()
    _dispatch.merged = (tiles_m.cpu().numpy(), int(ntiles_m[0]))
    return out


def _expected_tiles(offsets, E, TK, shared_rows, m_tile, grouped=False):
    """m_tile-row tiles of every group; those of more than m_tile / 2 rows first, then the short ones, each part in
    group order (grouped: all in group order)."""
    out = []
    for g in range(E + (1 if shared_rows else 0)):
        r0 = offsets[g] if g < E else TK
        n = (offsets[g + 1] - offsets[g]) if g < E else shared_rows
        for i in range(0, n, m_tile):
            out.append((g, r0 + i, r0 + min(n, i + m_tile), 0))
    if not grouped:
        out = [t for t in out if t[2] - t[1] > m_tile // 2] + [t for t in out if t[2] - t[1] <= m_tile // 2]
    return np.array(out, dtype=np.int32).reshape(-1, 4)


def _expected_merged(offsets, E, TK, shared_rows, m_tile, gkind, merge_rows):
    """The merged list: an int4-kind group's (gkind >> 16 == 0) last tile of at most merge_rows - m_tile rows joins
    the full tile before it; the merged tiles, then the other tiles of more than m_tile / 2 rows, then the shorter
    ones, each part in group order. Written from the rule itself, tile by tile."""
    merged, long_, short = [], [], []
    for g in range(E + (1 if shared_rows else 0)):
        r0 = offsets[g] if g < E else TK
        n = (offsets[g + 1] - offsets[g]) if g < E else shared_rows
        t = [(g, r0 + i, r0 + min(n, i + m_tile), gkind[g]) for i in range(0, n, m_tile)]
        if len(t) >= 2 and gkind[g] >> 16 == 0 and t[-1][2] - t[-1][1] <= merge_rows - m_tile:
            last = t.pop()
            full = t.pop()
            merged.append((g, full[1], last[2], gkind[g]))
        for x in t:
            (long_ if x[2] - x[1] > m_tile // 2 else short).append(x)
    return np.array(merged + long_ + short, dtype=np.int32).reshape(-1, 4)


def _zipf_topi(T, K, E, s, gen):
    p = 1.0 / np.arange(1, E + 1) ** s
    p /= p.sum()
    rng = np.random.default_rng(int(gen.initial_seed()))
    return np.stack([rng.choice(E, K, replace=False, p=p) for _ in range(T)]).astype(np.int64)


@pytest.mark.parametrize("T,K,E,shared,kind", [(4092, 8, 256, True, "uniform"), (128, 2, 8, True, "uniform"),
                                               (4096, 8, 256, False, "zipf"), (1, 8, 256, True, "uniform"),
                                               (0, 8, 256, True, "uniform"), (1000, 1, 3, False, "uniform"),
                                               (257, 4, 512, True, "zipf"),
                                               # 64 blocks of 1024 slots: the last size with the scan and the
                                               # scatter in one launch; 71 blocks: three launches
                                               (8192, 8, 128, False, "uniform"), (9000, 8, 256, True, "zipf")])
def test_dispatch_bitexact(T, K, E, shared, kind):
    _say(f"dispatch T{T} K{K} E{E} {kind}")
    gen = torch.Generator().manual_seed(T * 7 + E)
    if kind == "zipf":
        topi = _zipf_topi(T, K, E, 1.2, gen)
    else:
        topi = np.stack([torch.randperm(E, generator=gen)[:K].numpy() for _ in range(T)]) if T and K <= E else \
            np.zeros((T, K), np.int64)
        topi = topi.reshape(T, K).astype(np.int64)
    sh = T if shared else 0
    for dt in (torch.int32, torch.int64):
        # with int64 ids, also hand over group kinds: the tile list then carries them in its fourth field
        gkind = [(g * 7919) & 0x3ffff for g in range(E + 1)] if dt == torch.int64 else None
        counts, offsets, order, inv, tiles, ntiles, err = _dispatch(torch.from_numpy(topi).to(DEV, dt), T, K, E, sh,
                                                                    gkind=gkind, merge_rows=160 if gkind else 0)
        c0, o0, ord0, inv0 = intref.dispatch(topi, E)
        assert err[0] == 0
        assert np.array_equal(counts, c0) and np.array_equal(offsets, o0)
        if T:
            assert np.array_equal(order, ord0) and np.array_equal(inv, inv0)
        want = _expected_tiles(o0, E, T * K, sh, 128)
        want_g = _expected_tiles(o0, E, T * K, sh, 128, grouped=True)
        if gkind is not None:
            want[:, 3] = np.asarray(gkind, np.int32)[want[:, 0]]
            want_g[:, 3] = np.asarray(gkind, np.int32)[want_g[:, 0]]
        assert ntiles[0] == len(want)
        assert np.array_equal(tiles.reshape(-1, 4)[:len(want)], want)
        assert np.array_equal(_dispatch.grouped.reshape(-1, 4)[:len(want)], want_g)
        if gkind is not None:   # the merged list for the gate_up forward: every row in exactly one tile
            want_m = _expected_merged(o0, E, T * K, sh, 128, np.asarray(gkind, np.int32), 160)
            got_m, n_m = _dispatch.merged
            assert n_m == len(want_m) and np.array_equal(got_m.reshape(-1, 4)[:n_m], want_m)
            cover = np.zeros(T * K + sh, np.int32)
            for _, a, b, _k in want_m:
                cover[a:b] += 1
            assert (cover == 1).all()


def test_dispatch_flags_bad_ids():
    _say("dispatch bad ids")
    topi = torch.tensor([[0, 3], [9, 1], [2, -1]], dtype=torch.int64)
    counts, offsets, order, inv, tiles, ntiles, err = _dispatch(topi.to(DEV), 3, 2, 4)
    assert err[0] & 1
    assert counts.tolist() == [1, 1, 1, 1] and inv[2] == -1 and inv[5] == -1


# ------------------------------------------------------------------------------------------------- the MoE layer

LAYERS = {
    # name: make_layer kwargs
    "c1": dict(T=128, H=64, E=8, I=32, K=2, n_sel=2, r=4, alpha=8.0, shared_inter=32, group=64, down_group=32,
               lora_b_std=0.02),
    "mid": dict(T=300, H=256, E=16, I=128, K=4, n_sel=3, r=8, alpha=16.0, shared_inter=128, group=64,
                lora_b_std=0.05),
    "r16": dict(T=517, H=512, E=32, I=256, K=8, n_sel=4, r=16, alpha=32.0, shared_inter=256, group=64,
                lora_b_std=0.05),
    "frozen_only": dict(T=200, H=128, E=8, I=64, K=2, n_sel=0, r=0, shared_inter=64, group=64),
    "bf16_bank": dict(T=150, H=128, E=8, I=64, K=2, n_sel=2, r=4, alpha=8.0, shared_inter=64, int4=False,
                      lora_b_std=0.05),
    "no_shared": dict(T=190, H=128, E=8, I=64, K=2, n_sel=2, r=4, alpha=8.0, shared_inter=None, group=32,
                      lora_b_std=0.05),
    # a shared expert of another intermediate size than the experts' runs as its own GEMMs (smel/moe.py:197-201)
    "shared_wide": dict(T=300, H=256, E=16, I=128, K=4, n_sel=3, r=8, alpha=16.0, shared_inter=192, group=64,
                        lora_b_std=0.05),
    "shared_narrow": dict(T=260, H=128, E=8, I=128, K=2, n_sel=2, r=4, alpha=8.0, shared_inter=64, group=64,
                          lora_b_std=0.05),
    # more than 256 experts (the router's 8-logits-per-lane selection)
    "e512": dict(T=200, H=128, E=512, I=64, K=8, n_sel=3, r=4, alpha=8.0, shared_inter=64, group=64,
                 lora_b_std=0.05),
    # LoRA ranks above 16: the gate_up K-extension in two 32-wide planes (gate, up); mixed ranks in one launch (the
    # rank-8 shared set laid out in two planes too); a split shared expert with its own two-plane extension
    "r32": dict(T=400, H=256, E=16, I=128, K=4, n_sel=3, r=32, alpha=64.0, shared_inter=128, group=64,
                lora_b_std=0.05),
    "r24_mixed": dict(T=333, H=256, E=16, I=128, K=4, n_sel=4, r=24, alpha=48.0, shared_inter=128, group=64,
                      lora_b_std=0.05, r_shared=8),
    "r32_shared_split": dict(T=260, H=256, E=16, I=128, K=4, n_sel=2, r=32, alpha=32.0, shared_inter=192, group=64,
                             lora_b_std=0.05),
    # a rank that is not a multiple of 4: the LoRA gradients' stores of ragged rank groups and unaligned rows
    "r6": dict(T=280, H=256, E=16, I=128, K=4, n_sel=3, r=6, alpha=12.0, shared_inter=128, group=64,
               lora_b_std=0.05),
}


def run_layer(name, seed=0, gy_std=1e-2):
    from smel.moe import moe_forward
    kw = dict(LAYERS[name])
    x, ol = R.make_layer(seed=seed, **kw)
    W, ex, lora = to_device_layer(ol, DEV)
    xg = x.to(DEV).requires_grad_(True)
    seen = {}
    y = moe_forward(xg, W, ex, kw["K"], lora, stats=lambda p, v, i: seen.update(p=p.clone(), v=v.clone(), i=i.clone()))
    gy = (torch.randn(x.shape, generator=torch.Generator().manual_seed(seed + 1)) * gy_std).to(torch.bfloat16)
    y.backward(gy.to(DEV))
    torch.cuda.synchronize()
    grads = {}
    if lora is not None:
        for tag, m in (("ex", lora.experts), ("sh", lora.shared)):
            if m is not None:
                for n in LORA_NAMES:
                    grads[f"{tag}_{n}"] = getattr(m, n).grad.detach().cpu()
    return dict(x=x, ol=ol, gy=gy, y=y.detach().cpu(), dx=xg.grad.detach().cpu(), grads=grads,
                topi=seen["i"].cpu(), topv=seen["v"].cpu(), probs=seen["p"].cpu())


@pytest.mark.parametrize("name", list(LAYERS))
def test_layer_parity(name):
    _say(f"layer parity {name}")
    g = run_layer(name)
    K = LAYERS[name]["K"]
    # the oracle on the same bf16 inputs in fp32, forced to the kernel's routing
    y, dx, grads = R.moe_forward_backward(g["x"], g["ol"], K, g["gy"], forced_topi=g["topi"], dtype=torch.float32)
    assert_close_bf16(g["y"], y, "y")
    assert_close_bf16(g["dx"], dx, "dx")
    for k, v in grads.items():
        assert_close_bf16(g["grads"][k], v, k)
    assert set(grads) == set(g["grads"])


@pytest.mark.parametrize("name", ["r16"])
def test_merged_short_tiles_bitwise(name, monkeypatch):
    """The forward GEMMs' merged tiles (a full int4 tile and the expert's last tile of <= 32 rows in one block, on the
    dispatch's merged list: the gate_up and the down projection) accumulate every row in the same k order as the
    separate tiles: y, dX and the LoRA gradients are bitwise equal with and without the merge. (r16: 32 experts of
    about 129 rows, so most experts have a short last tile.)"""
    import smel.moe as M
    _say(f"merged short tiles {name}")
    monkeypatch.setattr(M, "_MERGE_SHORT", True)
    a = run_layer(name, seed=4)
    monkeypatch.setattr(M, "_MERGE_SHORT", False)
    b = run_layer(name, seed=4)
    counts = torch.bincount(a["topi"].flatten(), minlength=LAYERS[name]["E"])
    assert bool(((counts > 128) & (counts <= 160)).any()), counts   # some expert has a merged tile
    assert torch.equal(a["y"].view(torch.int16), b["y"].view(torch.int16))
    assert torch.equal(a["dx"].view(torch.int16), b["dx"].view(torch.int16))
    for k in b["grads"]:
        assert torch.equal(a["grads"][k], b["grads"][k]), k


@pytest.mark.parametrize("name", ["r16", "r24_mixed", "c1"])
def test_shared_lora_rows_on_side_stream_bitwise(name, monkeypatch):
    """The fused shared expert's gate_up LoRA rows projected on a side stream beside the router (SMEL_FWD_EXT_SIDE,
    token-order tiles written at rows TK + t) and the selected experts' rows after the dispatch give the same rows as
    one projection over the dispatch's tiles: y, dX and the LoRA gradients are bitwise equal. (r24_mixed: two planes;
    c1: T = 128, a single shared tile.)"""
    import smel.moe as M
    _say(f"shared LoRA rows on the side stream {name}")
    monkeypatch.setattr(M, "_FWD_EXT_SIDE", True)
    a = run_layer(name, seed=6)
    monkeypatch.setattr(M, "_FWD_EXT_SIDE", False)
    b = run_layer(name, seed=6)
    assert torch.equal(a["y"].view(torch.int16), b["y"].view(torch.int16))
    assert torch.equal(a["dx"].view(torch.int16), b["dx"].view(torch.int16))
    assert set(a["grads"]) == set(b["grads"]) and any(k.startswith("sh_") for k in b["grads"])
    for k in b["grads"]:
        assert torch.equal(a["grads"][k], b["grads"][k]), k


@pytest.mark.parametrize("name", ["r16", "r32", "shared_wide", "r24_mixed"])
def test_bwd_lora_rows_against_projection(name, monkeypatch):
    """The gate_up backward's LoRA rows from the down backward's per-column-block partials (smel_gmm_bwd_lr +
    smel_lora_rows_sum, the default) against the separate smel_lora_ext projection of dh: the same rows up to their
    bf16 rounding, so dX and every LoRA gradient agree far inside the bf16 bar (and both pass it against the oracle in
    test_layer_parity)."""
    import smel.moe as M
    _say(f"bwd LoRA rows vs projection {name}")
    monkeypatch.setattr(M, "_BWD_LORA_ROWS", True)
    a = run_layer(name, seed=3)
    monkeypatch.setattr(M, "_BWD_LORA_ROWS", False)
    b = run_layer(name, seed=3)
    assert torch.equal(a["y"].view(torch.int16), b["y"].view(torch.int16))
    assert_close_bf16(a["dx"], b["dx"], "dx", rel=5e-3, cos=0.99999)
    for k in b["grads"]:
        assert_close_bf16(a["grads"][k], b["grads"][k], k, rel=1e-2, cos=0.99999)


def test_layer_determinism():
    _say("determinism mid x3")
    runs = [run_layer("mid", seed=5) for _ in range(3)]
    for r in runs[1:]:
        assert torch.equal(r["y"].view(torch.int16), runs[0]["y"].view(torch.int16))
        assert torch.equal(r["dx"].view(torch.int16), runs[0]["dx"].view(torch.int16))
        for k in r["grads"]:
            assert torch.equal(r["grads"][k], runs[0]["grads"][k]), k


def test_routed_experts_parity():
    """routed_experts with routing given by the caller (the Gemma-4 call site, smel/layer_runner.py:258)."""
    from smel.moe import routed_experts
    _say("routed_experts")
    x, ol = R.make_layer(T=211, H=256, E=16, I=128, K=4, n_sel=3, r=8, alpha=16.0, shared_inter=None, seed=2,
                         lora_b_std=0.05)
    W, ex, lora = to_device_layer(ol, DEV)
    probs, topv, topi = R.route(x.float(), ol.gate_w.float(), 4)
    tv = topv.to(torch.bfloat16)
    xg = x.to(DEV).requires_grad_(True)
    tvg = tv.to(DEV).float().requires_grad_(True)
    y = routed_experts(xg, tvg, topi.to(DEV), ex, lora.experts)
    gy = (torch.randn(x.shape, generator=torch.Generator().manual_seed(9)) * 1e-2).to(torch.bfloat16)
    y.backward(gy.to(DEV))
    # oracle
    xo = x.float().requires_grad_(True)
    tvo = tv.float().requires_grad_(True)
    leaves = {n: ol.ex_lora[n].clone().requires_grad_(True) for n in LORA_NAMES}
    yo = R.routed_experts(xo, tvo, topi, ol, leaves, torch.float32)
    yo.backward(gy.float())
    assert_close_bf16(y.detach().cpu(), yo.detach(), "y")
    assert_close_bf16(xg.grad.cpu(), xo.grad, "dx")
    assert_close_bf16(tvg.grad.cpu(), tvo.grad, "dtopv")
    for n in LORA_NAMES:
        assert_close_bf16(getattr(lora.experts, n).grad.cpu(), leaves[n].grad, n)


def test_routed_experts_bad_ids():
    """Expert ids outside [0, E) given to routed_experts (the reference's bincount / indexing fails there): the call
    itself does not synchronise; its dispatch drops those slots (zero rows: the output equals the oracle's with those
    routing weights set to zero, no uninitialised rows are read) and the error is raised by check_routing_errors() or,
    once the call's check has landed, by the next call. Under HIP-graph capture nothing is reported and the replays
    drop the slots the same way."""
    from smel.moe import check_routing_errors, routed_experts
    _say("routed_experts bad ids")
    x, ol = R.make_layer(T=96, H=128, E=8, I=64, K=2, n_sel=2, r=4, alpha=8.0, shared_inter=None, seed=8,
                         lora_b_std=0.05)
    W, ex, lora = to_device_layer(ol, DEV)
    probs, topv, topi = R.route(x.float(), ol.gate_w.float(), 2)
    bad = topi.clone()
    bad[3, 1], bad[40, 0], bad[77, 1] = 8, -1, 1000
    xd, tvd, bd = x.to(DEV), topv.float().to(DEV), bad.to(DEV)
    keep = (bad >= 0) & (bad < 8)
    tv0 = torch.where(keep, topv.float(), torch.zeros_like(topv.float()))
    ids0 = torch.where(keep, bad, torch.zeros_like(bad))
    yo = R.routed_experts(x.float(), tv0, ids0, ol, {n: ol.ex_lora[n].clone() for n in LORA_NAMES}, torch.float32)
    with torch.no_grad():
        for _ in range(4):   # calls back to back: the earlier checks may still be in flight when the next polls
            routed_experts(xd, tvd, topi.to(DEV), ex, lora.experts)
        check_routing_errors()
        y_eager = routed_experts(xd, tvd, bd, ex, lora.experts)   # returns without waiting for the check
    with pytest.raises(IndexError):
        check_routing_errors()
    check_routing_errors()                                           # reported once
    assert_close_bf16(y_eager.cpu(), yo, "y (eager, bad ids dropped)")
    with torch.no_grad():
        routed_experts(xd, tvd, bd, ex, lora.experts)
        torch.cuda.synchronize()                                     # the check has landed: the next call raises
        with pytest.raises(IndexError):
            routed_experts(xd, tvd, topi.to(DEV), ex, lora.experts)
    check_routing_errors()
    with torch.no_grad():
        routed_experts(xd, tvd, topi.to(DEV), ex, lora.experts)    # warm-up: packs and caches outside the capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            y = routed_experts(xd, tvd, bd, ex, lora.experts)
        for _ in range(2):
            g.replay()
            torch.cuda.synchronize()
            assert torch.isfinite(y.float()).all()
            assert_close_bf16(y.cpu(), yo, "y")
    check_routing_errors()   # captured calls record nothing


def test_route_api_backward():
    """route() alone: d topv flows back to x through renorm + softmax + the router GEMM."""
    from smel.moe import route
    _say("route api backward")
    gen = torch.Generator().manual_seed(4)
    T, H, E, K = 130, 128, 32, 4
    x = torch.randn(T, H, generator=gen).to(torch.bfloat16)
    gw = (torch.randn(E, H, generator=gen) * 0.05).to(torch.bfloat16)
    xg = x.to(DEV).requires_grad_(True)
    probs, topv, topi = route(xg, gw.to(DEV), K)
    cot = torch.randn(T, K, generator=gen)
    (topv.float() * cot.to(DEV)).sum().backward()
    xo = x.float().requires_grad_(True)
    lo = xo @ gw.float().t()
    po = torch.softmax(lo, -1)
    sel = po.gather(1, topi.cpu())
    tvo = sel / sel.sum(-1, keepdim=True)
    (tvo * cot).sum().backward()
    assert_close_bf16(xg.grad.cpu(), xo.grad, "dx", rel=3e-2, cos=0.999)


@pytest.mark.parametrize("act_name,T,H,Is,r", [("silu", 300, 256, 128, 8), ("gelu_tanh", 257, 512, 192, 16),
                                               ("silu", 64, 128, 64, 0), ("gelu_tanh", 190, 256, 128, 32),
                                               ("silu", 140, 128, 64, 20)])
def test_mlp_lora_parity(act_name, T, H, Is, r):
    """mlp_lora (smel/moe.py:183-194; Gemma-4's dense GeGLU MLP with act gelu_tanh) as the dense group."""
    from smel.lora import MLPLoRA
    from smel.moe import mlp_lora
    _say(f"mlp_lora {act_name} T{T} H{H} Is{Is} r{r}")
    gen = torch.Generator().manual_seed(T)
    x = torch.randn(T, H, generator=gen).to(torch.bfloat16)
    wg = (torch.randn(Is, H, generator=gen) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(Is, H, generator=gen) * 0.02).to(torch.bfloat16)
    wd = (torch.randn(H, Is, generator=gen) * 0.02).to(torch.bfloat16)
    lora = None
    if r:
        lora = MLPLoRA(H, Is, r, 2.0 * r)
        with torch.no_grad():
            for n in ("B_gate", "B_up", "B_down"):
                getattr(lora, n).copy_(torch.randn(getattr(lora, n).shape, generator=gen) * 0.05)
        lora = lora.to(DEV)
    xg = x.to(DEV).requires_grad_(True)
    y = mlp_lora(xg, wg.to(DEV), wu.to(DEV), wd.to(DEV), lora, act_name)
    gy = (torch.randn(T, H, generator=gen) * 1e-2).to(torch.bfloat16)
    y.backward(gy.to(DEV))
    xo = x.float().requires_grad_(True)
    L_o = {n: getattr(lora, n).detach().cpu().clone().requires_grad_(True) for n in LORA_NAMES} if r else None
    yo = R.mlp_lora(xo, torch.cat((wg, wu)).float(), wd.float(), L_o, 2.0 if r else 0.0, act_name)
    yo.backward(gy.float())
    assert_close_bf16(y.detach().cpu(), yo.detach(), "y")
    assert_close_bf16(xg.grad.cpu(), xo.grad, "dx")
    if r:
        for n in LORA_NAMES:
            assert_close_bf16(getattr(lora, n).grad.cpu(), L_o[n].grad, n)


def test_gelu_experts_parity():
    """GELU-tanh routed experts (Gemma 4's act, smel/moe.py:91-107) through routed_experts."""
    from smel.moe import routed_experts
    _say("gelu experts")
    x, ol = R.make_layer(T=180, H=256, E=16, I=128, K=4, n_sel=2, r=8, alpha=16.0, shared_inter=None, seed=6,
                         act_name="gelu_tanh", lora_b_std=0.05)
    W, ex, lora = to_device_layer(ol, DEV)
    probs, topv, topi = R.route(x.float(), ol.gate_w.float(), 4)
    tv = topv.to(torch.bfloat16)
    xg = x.to(DEV).requires_grad_(True)
    y = routed_experts(xg, tv.to(DEV), topi.to(DEV), ex, lora.experts)
    gy = (torch.randn(x.shape, generator=torch.Generator().manual_seed(2)) * 1e-2).to(torch.bfloat16)
    y.backward(gy.to(DEV))
    xo = x.float().requires_grad_(True)
    leaves = {n: ol.ex_lora[n].clone().requires_grad_(True) for n in LORA_NAMES}
    yo = R.routed_experts(xo, tv.float(), topi, ol, leaves, torch.float32)
    yo.backward(gy.float())
    assert_close_bf16(y.detach().cpu(), yo.detach(), "y")
    assert_close_bf16(xg.grad.cpu(), xo.grad, "dx")
    for n in LORA_NAMES:
        assert_close_bf16(getattr(lora.experts, n).grad.cpu(), leaves[n].grad, n)


@pytest.mark.parametrize("int4,act_name,counts", [
    (True, "silu", [9, 0, 12, 7, 15, 7]),                        # the reference's own counts (test_gemma4.py:157)
    (False, "gelu_tanh", [9, 0, 12, 7, 15, 7]),
    (True, "silu", [0, 300, 1, 129, 0, 0, 64, 128]),              # tiles split at 128 rows, empty experts
    (True, "gelu_tanh", [0, 0, 0, 0, 0, 0]),                      # no rows at all
    # full tiles merged with a last tile of <= 32 rows in the gate_up forward (160, 129, 150, 288 = 128 + 160),
    # and not merged (161 = 128 + 33, 96)
    (True, "silu", [160, 0, 129, 161, 288, 5, 150, 96]),
])
def test_frozen_experts_fn(int4, act_name, counts):
    """FrozenExpertsFn.apply(xs, counts, bank, group, act) (smel/moe.py:120-143) on rows sorted by expert, forward
    and dX, against the oracle's restatement of the reference's per-group dequant / recompute backward."""
    from smel.moe import FrozenExpertsFn
    E = len(counts)
    _say(f"FrozenExpertsFn int4={int4} {act_name} counts={counts}")
    _, ol = R.make_layer(T=8, H=128, E=E, I=64, K=1, int4=int4, act_name=act_name, seed=11)
    _, bank_dev, _ = to_device_layer(ol, DEV)
    bank = bank_dev.frozen
    N = sum(counts)
    gen = torch.Generator().manual_seed(N + E)
    xs = torch.randn(N, 128, generator=gen).to(torch.bfloat16)
    gy = (torch.randn(N, 128, generator=gen) * 1e-2).to(torch.bfloat16)
    xg = xs.to(DEV).requires_grad_(True)
    y = FrozenExpertsFn.apply(xg, counts, bank, 2, act_name)
    y.backward(gy.to(DEV))
    torch.cuda.synchronize()
    assert y.shape == (N, 128) and xg.grad.shape == (N, 128)
    if N == 0:
        return
    xo = xs.float().requires_grad_(True)
    yo = R._FrozenExperts.apply(xo, counts, ol, torch.float32)
    yo.backward(gy.float())
    assert_close_bf16(y.detach().cpu(), yo.detach(), "y")
    assert_close_bf16(xg.grad.cpu(), xo.grad, "dx")


# ------------------------------------------------------------------------------------------------- Gemma 4 router


def _gemma_router_inputs(T, H, E, seed):
    gen = torch.Generator().manual_seed(seed)
    h = (torch.randn(T, H, generator=gen) * 3.0).to(torch.bfloat16)                 # residual stream
    W = {"router.scale": (1.0 + 0.2 * torch.randn(H, generator=gen)).to(torch.bfloat16),   # tiny.py:74-77
         "router.proj.weight": (torch.randn(E, H, generator=gen) * 0.5).to(torch.bfloat16),
         "router.per_expert_scale": (0.5 + torch.rand(E, generator=gen)).to(torch.bfloat16)}
    return h, W


@pytest.mark.parametrize("T,H,E,K", [(4096, 2816, 128, 8), (128, 64, 8, 2), (333, 256, 32, 4), (1, 128, 256, 16)])
def test_route_gemma4_forward(T, H, E, K):
    """smel_route_gemma4 (smel/moe.py:170-180): the router input xn against the oracle's bf16 roundings (at most two
    bf16 ulps apart, where the fp32 rstd of the two differs in its last bits), the logits within bf16 tolerance, and
    probs / topv / ids bit-for-bit what the oracle's selection gives on the kernel's own logits."""
    L = _lib()
    _say(f"route_gemma4 T{T} H{H} E{E} K{K}")
    eps = 1e-6
    h, W = _gemma_router_inputs(T, H, E, T + H)
    d = {k: v.to(DEV) for k, v in W.items()}
    hd = h.to(DEV)
    f = lambda *s, dt=torch.float32: torch.empty(*s, dtype=dt, device=DEV)
    probs, topv, topi, topi32 = f(T, E), f(T, K), f(T, K, dt=torch.int64), f(T, K, dt=torch.int32)
    xn, rstd = f(T, H, dt=torch.bfloat16), f(T)
    ldl = L.load().smel_route_ld(E, 0)
    lg = f(T, ldl, dt=torch.bfloat16)
    L.call("smel_route_gemma4", L.ptr(hd), L.ptr(d["router.scale"]), L.ptr(d["router.proj.weight"]),
           L.ptr(d["router.per_expert_scale"]), T, H, E, K, eps, L.ptr(probs), L.ptr(topv), L.ptr(topi),
           L.ptr(topi32), L.ptr(xn), L.ptr(rstd), L.ptr(lg), L.stream())
    torch.cuda.synchronize()
    # router input: the oracle's expression on the CPU
    hf = h.float()
    r = torch.pow(hf.pow(2).mean(-1, keepdim=True) + eps, -0.5)
    xo = (hf * r).to(torch.bfloat16) * W["router.scale"] * H ** -0.5
    assert torch.allclose(rstd.cpu(), r[:, 0], rtol=1e-6, atol=0)
    diff = (xn.cpu().float() - xo.float()).abs()
    ulp = xo.float().abs() * 2 ** -6
    assert bool((diff <= ulp + 1e-30).all())
    assert (diff > 0).float().mean().item() < 1e-3
    # logits of the kernel's own xn: fp32-accumulated dot products, rounded once
    lref = (xn.cpu().double() @ W["router.proj.weight"].double().t())
    glog = lg.cpu().float()[:, :E]
    assert torch.allclose(glog.double(), lref, rtol=1e-2, atol=1e-2)
    # selection on identical logits: the oracle's softmax / top-k / renorm / per-expert scale
    po = torch.softmax(glog, -1, dtype=torch.float32)
    vo, io = R.topk_lowest_index(po, K)
    assert torch.equal(topi.cpu(), io) and torch.equal(topi32.cpu().long(), io)
    to = vo / vo.sum(-1, keepdim=True) * W["router.per_expert_scale"][io]
    assert torch.allclose(probs.cpu(), po, rtol=1e-5, atol=1e-7)
    assert torch.allclose(topv.cpu(), to, rtol=1e-5, atol=1e-7)


def test_route_gemma4_backward():
    """route_gemma4 through the API: d topv flows back to h through the per-expert scale, renorm, softmax, router
    GEMM, the two bf16 scalings and the weightless RMSNorm; vs fp32 autograd of the reference formula, same ids."""
    from smel.moe import route_gemma4
    _say("route_gemma4 backward")
    T, H, E, K, eps = 200, 256, 32, 4, 1e-6
    h, W = _gemma_router_inputs(T, H, E, 21)
    hg = h.to(DEV).requires_grad_(True)
    probs, topv, topi = route_gemma4(hg, {k: v.to(DEV) for k, v in W.items()}, K, eps)
    assert topv.dtype == torch.float32 and probs.dtype == torch.float32 and topi.dtype == torch.int64
    cot = torch.randn(T, K, generator=torch.Generator().manual_seed(3))
    (topv * cot.to(DEV)).sum().backward()
    ho = h.float().requires_grad_(True)
    r = torch.pow(ho.pow(2).mean(-1, keepdim=True) + eps, -0.5)
    x = ho * r * W["router.scale"].float() * H ** -0.5
    po = torch.softmax(x @ W["router.proj.weight"].float().t(), -1)
    ti = topi.cpu()
    sel = po.gather(1, ti)
    tvo = sel / sel.sum(-1, keepdim=True) * W["router.per_expert_scale"].float()[ti]
    (tvo * cot).sum().backward()
    assert torch.allclose(topv.detach().cpu(), tvo.detach(), rtol=3e-2, atol=1e-3)
    assert_close_bf16(hg.grad.cpu(), ho.grad, "dh", rel=3e-2, cos=0.999)


# ------------------------------------------------------------------------------------------ skewed routing (C5 kind)


def _skewed_layer(seed=0):
    """A layer whose router prefers a few experts (Zipf(1.2) logit bias through the inputs, as bench.py's C5 does):
    hot experts span many 128-row tiles, some experts get no rows; the 4 most popular are the selected ones."""
    T, H, E, I, K = 1500, 256, 32, 128, 4
    x, ol = R.make_layer(T=T, H=H, E=E, I=I, K=K, n_sel=0, r=8, alpha=16.0, shared_inter=I, seed=seed,
                         lora_b_std=0.05)
    g = torch.Generator().manual_seed(seed + 100)
    perm = torch.randperm(E, generator=g)
    rank = torch.empty(E, dtype=torch.long)
    rank[perm] = torch.arange(E)
    bias = -1.2 * 0.6 * torch.log(rank.double() + 1.0)
    gw = ol.gate_w.float()
    ol.gate_w = (gw - gw.mean(1, keepdim=True) + (bias / H).float()[:, None]).to(torch.bfloat16)
    x = (x.float() + 1.0).to(torch.bfloat16)
    sel = perm[:4].tolist()
    # selected experts: bf16 copies of the bank's dequantized weights + LoRA
    wgu, wdn = ol.frozen_weights(0, E, torch.float32)
    ol.sel_ids = sel
    ol.sel_gate_up, ol.sel_down = wgu[sel].to(torch.bfloat16), wdn[sel].to(torch.bfloat16)
    ex_l = {}
    for n, shp, fan in (("A_gate", (4, 8, H), H), ("A_up", (4, 8, H), H), ("A_down", (4, 8, I), I)):
        ex_l[n] = (torch.rand(*shp, generator=g) * 2 - 1) / fan ** 0.5
    for n, shp in (("B_gate", (4, I, 8)), ("B_up", (4, I, 8)), ("B_down", (4, H, 8))):
        ex_l[n] = torch.randn(*shp, generator=g) * 0.05
    ol.ex_lora, ol.ex_scale = ex_l, 2.0
    return x, ol, K


def test_layer_skewed_parity_and_determinism():
    from smel.moe import moe_forward
    _say("skewed routing layer")
    x, ol, K = _skewed_layer()
    W, ex, lora = to_device_layer(ol, DEV)
    gy = (torch.randn(x.shape, generator=torch.Generator().manual_seed(5)) * 1e-2).to(torch.bfloat16)
    outs = []
    for _ in range(3):
        xg = x.to(DEV).requires_grad_(True)
        for m in (lora.experts, lora.shared):
            for n in LORA_NAMES:
                getattr(m, n).grad = None
        seen = {}
        y = moe_forward(xg, W, ex, K, lora, stats=lambda p, v, i: seen.update(i=i.clone()))
        y.backward(gy.to(DEV))
        torch.cuda.synchronize()
        grads = {f"{t}_{n}": getattr(m, n).grad.detach().cpu().clone() for t, m in (("ex", lora.experts),
                                                                                    ("sh", lora.shared))
                 for n in LORA_NAMES}
        outs.append((y.detach().cpu(), xg.grad.cpu(), grads, seen["i"].cpu()))
    counts = torch.bincount(outs[0][3].reshape(-1), minlength=32)
    _say(f"  rows per expert: max {int(counts.max())}, min {int(counts.min())}, empty {int((counts == 0).sum())}")
    assert int(counts.max()) > 3 * 128          # hot experts span several tiles
    for o in outs[1:]:                           # bitwise repeatable
        assert torch.equal(o[0].view(torch.int16), outs[0][0].view(torch.int16))
        assert torch.equal(o[1].view(torch.int16), outs[0][1].view(torch.int16))
        for k in o[2]:
            assert torch.equal(o[2][k], outs[0][2][k]), k
    y, dx, grads = R.moe_forward_backward(x, ol, K, gy, forced_topi=outs[0][3], dtype=torch.float32)
    assert_close_bf16(outs[0][0], y, "y")
    assert_close_bf16(outs[0][1], dx, "dx")
    for k, v in grads.items():
        assert_close_bf16(outs[0][2][k], v, k)
