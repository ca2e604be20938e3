"""MoE layer of SMEL FT on MI355X kernels: the public API of the reference's smel/moe.py (drop-in for its callers,
smel/layer_runner.py:243-291), every step a HIP kernel of libsmel_moe.so reached through the C-ABI.

Forward (``moe_forward``): router (logits + softmax + top-k + renorm, and the shared-expert gate logit) -> stats hook ->
stable counting-sort dispatch (device-side tile list, no host sync) -> LoRA down-projections of LoRA rows ->
grouped gate_up GEMM (int4 dequant in registers / bf16 + LoRA K-extension, token gather fused, SiLU-gate epilogue)
-> grouped down GEMM -> fixed-order fp32 combine of the K slots and the shared expert. The shared expert is the
extra group E of the same grouped GEMMs (rows [TK, TK+T)).

Backward: down-backward GEMM fused with the SiLU-gate backward, the topv / shared-gate scaling and the d(weight)
partials -> gate_up-backward GEMM (int4 re-dequantized) -> router backward (renorm + softmax + shared gate) as a GEMM
against the router weight -> fixed-order dX reduce; LoRA dA / dB as fixed-order row reductions. Bitwise
run-to-run deterministic: no atomics anywhere.

Differences from the reference's rounding points (all inside the bf16 tolerance): the LoRA scale is folded into the
bf16 rank-r activations; LoRA terms accumulate in the same fp32 accumulator as the base GEMM; the combine adds the
shared expert in fp32 before the single rounding; gradients are accumulated in fp32.
"""
from __future__ import annotations

import ctypes
import os
from collections import OrderedDict

import torch
import torch.nn.functional as F

from . import _lib as L
from . import moe_f32 as F32
from .quant import dequant_int4, quantize_int4

M_TILE = 128      # rows per GEMM tile (the tile list of smel_dispatch)
M_MERGED = 160    # rows of a merged gate_up forward tile (a full tile + an int4 expert's last tile of <= 32 rows)
EXT = 32          # width of one plane of the LoRA K-extension
MAX_LORA_RANK = 32


def _lora_planes(*sets) -> int:
    """32-wide K-extension planes of the gate_up side for the LoRA sets one launch serves: one (gate and up packed,
    ranks 0..15 / 16..31: rank <= 16) or two (gate in plane 0, up in plane 1: rank <= 32). The down side always has
    one plane."""
    r = max((m.r for m in sets if m is not None), default=0)
    if r > MAX_LORA_RANK:
        raise L.SmelError(f"LoRA rank {r} is above the kernels' {MAX_LORA_RANK}")
    return 2 if r > EXT // 2 else 1
_ACT = {"silu": 0, "gelu_tanh": 1}
_GELU_C = 0.7978845608028654


# ------------------------------------------------------------------------------------------------ weight layouts


class PackedW:
    """One bf16 weight matrix [R, C] (or a stack of them, R rows each) in the GEMMs' fragment layout
    (smel_pack_bf16): ``t`` holds the packed bytes, ``R``/``C`` the shape of one matrix."""

    __slots__ = ("t", "R", "C")

    def __init__(self, t: torch.Tensor, R: int, C: int):
        self.t, self.R, self.C = t, R, C


def pack_bf16(*mats: torch.Tensor) -> PackedW:
    """Pack bf16 matrices [..., R_i, C] (same C) stacked along rows into one fragment-layout buffer; every part but
    the last needs a multiple of 32 rows. One matrix of the result has the rows of the last dimension-2 extent, i.e.
    a [E, R, C] bank packs as E matrices of R rows, and pack_bf16(gate, up) as one [2I, C] matrix."""
    C = mats[0].shape[-1]
    rows = [m.numel() // C for m in mats]
    if any(r % 32 for r in rows[:-1]):
        raise ValueError("pack_bf16: every part but the last needs a multiple of 32 rows")
    lib = L.load()
    total = sum(rows)
    out = torch.empty(lib.smel_packed_bytes(L.PACK_BF16, total, C) // 2, dtype=torch.bfloat16,
                      device=mats[0].device)
    off = 0
    for m, r in zip(mats, rows):
        m = _bf16(m)
        dst = out.data_ptr() + lib.smel_packed_bytes(L.PACK_BF16, off, C)
        L.call("smel_pack_bf16", L.ptr(m), r, C, C, dst, L.stream())
        off += r
    R = total if len(mats) > 1 else mats[0].shape[-2]
    return PackedW(out, R, C)


def pack_bf16_t(w: torch.Tensor) -> PackedW:
    """Pack bf16 matrices [..., R, C] (a [E, R, C] bank: E matrices) into the backward GEMM's transposed fragment
    layout (smel_pack_bf16_t)."""
    w = _bf16(w)
    R, C = w.shape[-2], w.shape[-1]
    n = w.numel() // (R * C)
    lib = L.load()
    out = torch.empty(lib.smel_packed_t_bytes(L.PACK_BF16, n, R, C, 0) // 2, dtype=torch.bfloat16, device=w.device)
    L.call("smel_pack_bf16_t", L.ptr(w), n, R, C, C, L.ptr(out), L.stream())
    return PackedW(out, R, C)


_PACK_CACHE: "OrderedDict" = OrderedDict()
_PACK_CACHE_MAX = 32


def _cached(kind: str, build, *mats: torch.Tensor, store: dict | None = None):
    """Packed form of per-call weights (shared expert, router, dense MLP) reused while the source tensors are
    unchanged: keyed by storage address, shape and strides, valid while the version counters (bumped by any in-place
    write, views included) are the ones it was built at. ``store``: the layer's own dict (LayerExperts), whose
    entries live and die with the layer and are replaced when their sources change; without one, a process-wide LRU
    of _PACK_CACHE_MAX entries. An entry holds its sources, so their addresses cannot be reused while it lives."""
    key = (kind,) + tuple((m.data_ptr(), tuple(m.shape), tuple(m.stride()), str(m.device)) for m in mats)
    ver = tuple(m._version for m in mats)
    cache = _PACK_CACHE if store is None else store
    hit = cache.get(key)
    if hit is not None and hit[0] == ver:
        if store is None:
            _PACK_CACHE.move_to_end(key)
        return hit[2]
    val = build()
    if store is not None and hit is None and len(store) >= _PACK_CACHE_MAX:
        store.clear()   # a layer called with ever new weight tensors keeps only the latest packs
    cache[key] = (ver, mats, val)
    if store is None:
        _PACK_CACHE.move_to_end(key)
        while len(_PACK_CACHE) > _PACK_CACHE_MAX:
            _PACK_CACHE.popitem(last=False)
    return val


# ------------------------------------------------------------------------------------------------ expert banks


class BF16Experts:
    """Frozen experts as fused 3-D tensors: gate_up [E, 2I, H], down [E, H, I] (smel/moe.py:18-32)."""

    def __init__(self, gate_up: torch.Tensor, down: torch.Tensor):
        self.gate_up, self.down = gate_up, down
        self.num_experts = gate_up.shape[0]

    def weights(self, e0: int, e1: int):
        return self.gate_up[e0:e1], self.down[e0:e1]

    def packed(self, which: str) -> PackedW:
        """gate_up ('gu') or down ('dn') in the GEMMs' fragment layout, built once (the bank is frozen)."""
        cache = self.__dict__.setdefault("_packed", {})
        if which not in cache:
            cache[which] = pack_bf16(_bf16(self.gate_up if which == "gu" else self.down))
        return cache[which]

    def packed_t(self, which: str) -> PackedW:
        """The same in the backward GEMM's transposed layout, built once."""
        cache = self.__dict__.setdefault("_packed_t", {})
        if which not in cache:
            cache[which] = pack_bf16_t(self.gate_up if which == "gu" else self.down)
        return cache[which]

    def tensors(self):
        return {"gate_up": self.gate_up, "down": self.down}

    def nbytes(self):
        return sum(t.numel() * t.element_size() for t in self.tensors().values())


class Int4Experts:
    """Frozen experts in group-wise int4 (smel/moe.py:35-55): dicts {"q", "scale", "zero"} for gate_up and down.
    The grouped GEMMs read this format directly; ``weights`` (bf16 copies) exists for API compatibility only."""

    def __init__(self, gu: dict, dn: dict, dtype=torch.bfloat16):
        self.gu, self.dn, self.dtype = gu, dn, dtype
        self.num_experts = gu["q"].shape[0]

    @classmethod
    def from_bf16(cls, gate_up, down, group=64):
        return cls(quantize_int4(gate_up, group), quantize_int4(down, group), dtype=gate_up.dtype)

    @staticmethod
    def group_of(d: dict) -> int:
        return d["q"].shape[-1] * 2 // d["scale"].shape[-1]

    def packed(self, which: str):
        """(q, scale/zero) of 'gu' or 'dn' in the GEMMs' fragment layout (smel_pack_int4), built once per bank: the
        bank is frozen (rebuild by deleting ``_packed`` after changing its tensors)."""
        cache = self.__dict__.setdefault("_packed", {})
        if which not in cache:
            d = self.gu if which == "gu" else self.dn
            E, R, half = d["q"].shape
            K = half * 2
            lib = L.load()
            qf = torch.empty(lib.smel_packed_bytes(L.PACK_Q4, E * R, K), dtype=torch.uint8, device=d["q"].device)
            szf = torch.empty(lib.smel_packed_bytes(L.PACK_SZ, E * R, K) // 4, dtype=torch.int32,
                              device=d["q"].device)
            L.call("smel_pack_int4", L.ptr(d["q"]), L.ptr(d["scale"]), L.ptr(d["zero"]), E * R, K,
                   Int4Experts.group_of(d), L.ptr(qf), L.ptr(szf), L.stream())
            cache[which] = (qf, szf)
        return cache[which]

    def fast_dq(self, which: str) -> bool:
        """Whether every scale/zero group of 'gu' or 'dn' admits the GEMMs' cheaper exact dequant form
        (smel_int4_fast_ok; checked once per bank, one host sync)."""
        cache = self.__dict__.setdefault("_fast_dq", {})
        if which not in cache:
            d = self.gu if which == "gu" else self.dn
            ok = torch.zeros(1, dtype=torch.int32, device=d["q"].device)
            L.call("smel_int4_fast_ok", L.ptr(d["scale"]), L.ptr(d["zero"]), d["scale"].numel(), L.ptr(ok),
                   L.stream())
            cache[which] = bool(ok.item())
        return cache[which]

    def packed_t(self, which: str):
        """(q, scale/zero) of 'gu' or 'dn' in the backward GEMM's transposed layout (smel_pack_int4_t), built once
        per bank: one more int4 copy (not a bf16 one) that the backward streams straight into registers; its
        scale/zero are fp32 pairs (zero pre-shifted for the fast dequant form when fast_dq holds)."""
        cache = self.__dict__.setdefault("_packed_t", {})
        if which not in cache:
            d = self.gu if which == "gu" else self.dn
            E, R, half = d["q"].shape
            C = half * 2
            g = Int4Experts.group_of(d)
            lib = L.load()
            qt = torch.empty(lib.smel_packed_t_bytes(L.PACK_Q4, E, R, C, g), dtype=torch.uint8, device=d["q"].device)
            szt = torch.empty(lib.smel_packed_t_bytes(L.PACK_SZ, E, R, C, g) // 4, dtype=torch.float32,
                              device=d["q"].device)
            L.call("smel_pack_int4_t", L.ptr(d["q"]), L.ptr(d["scale"]), L.ptr(d["zero"]), E, R, C, g,
                   int(self.fast_dq(which)), L.ptr(qt), L.ptr(szt), L.stream())
            cache[which] = (qt, szt)
        return cache[which]

    def weights(self, e0: int, e1: int):
        gu = dequant_int4(self.gu["q"][e0:e1], self.gu["scale"][e0:e1], self.gu["zero"][e0:e1], self.dtype)
        dn = dequant_int4(self.dn["q"][e0:e1], self.dn["scale"][e0:e1], self.dn["zero"][e0:e1], self.dtype)
        return gu, dn

    def tensors(self):
        return {f"gate_up.{k}": v for k, v in self.gu.items()} | {f"down.{k}": v for k, v in self.dn.items()}

    def nbytes(self):
        return sum(t.numel() * t.element_size() for t in self.tensors().values())


class LayerExperts:
    """Routed experts of one layer (smel/moe.py:146-159): the frozen bank for all E experts plus trainable bf16
    copies of the selected experts, whose bank copy is then ignored."""

    def __init__(self, frozen, sel_ids=None, sel_gate_up=None, sel_down=None, group: int = 32, act: str = "silu"):
        self.frozen = frozen
        self.E = frozen.num_experts
        self.group = group          # the reference's experts-dequantized-at-once knob; the kernels need none
        self.act = act
        self.sel_ids = None if sel_ids is None else torch.as_tensor(sel_ids, dtype=torch.long)
        self.sel_gate_up, self.sel_down = sel_gate_up, sel_down
        self._slot = {}
        if self.sel_ids is not None:
            self._slot = {int(e): j for j, e in enumerate(self.sel_ids.tolist())}
        self._gkind = {}

    def packed_sel(self):
        """(gate_up, down) of the selected experts in the GEMMs' fragment layout, built once (frozen base weights;
        their LoRA is applied on top). None without selected experts."""
        if self.sel_ids is None or not self._slot:
            return None
        if "_packed_sel" not in self.__dict__:
            self._packed_sel = (pack_bf16(_bf16(self.sel_gate_up)), pack_bf16(_bf16(self.sel_down)))
        return self._packed_sel

    def packed_sel_t(self):
        """The same in the backward GEMM's transposed layout, built once."""
        if self.sel_ids is None or not self._slot:
            return None
        if "_packed_sel_t" not in self.__dict__:
            self._packed_sel_t = (pack_bf16_t(self.sel_gate_up), pack_bf16_t(self.sel_down))
        return self._packed_sel_t

    def gkind(self, with_shared: bool, device) -> torch.Tensor:
        """Per-group weight location: (kind << 16) | index, groups 0..E-1 (+ E = shared)."""
        key = (with_shared, str(device))
        if key not in self._gkind:
            int4 = isinstance(self.frozen, Int4Experts)
            k = []
            for e in range(self.E):
                if e in self._slot:
                    k.append((L.KIND_SEL << 16) | self._slot[e])
                else:
                    k.append(((L.KIND_INT4 if int4 else L.KIND_BF16) << 16) | e)
            if with_shared:
                k.append(L.KIND_SHARED << 16)
            self._gkind[key] = torch.tensor(k, dtype=torch.int32, device=device)
        return self._gkind[key]


# ------------------------------------------------------------------------------------------------ activations


def act(x: torch.Tensor, name: str) -> torch.Tensor:
    """smel/moe.py:91-96 (elementwise helper of the API; the kernels fuse their own)."""
    if name == "silu":
        return F.silu(x)
    if name == "gelu_tanh":
        return F.gelu(x, approximate="tanh")
    raise ValueError(f"unknown activation {name}")


def act_and_grad(g: torch.Tensor, name: str):
    """smel/moe.py:99-107."""
    if name == "silu":
        sg = torch.sigmoid(g)
        return g * sg, sg * (1 + g * (1 - sg))
    if name == "gelu_tanh":
        t = torch.tanh(_GELU_C * (g + 0.044715 * g ** 3))
        return 0.5 * g * (1 + t), 0.5 * (1 + t) + 0.5 * g * (1 - t * t) * _GELU_C * (1 + 3 * 0.044715 * g * g)
    raise ValueError(f"unknown activation {name}")


# ------------------------------------------------------------------------------------------------ helpers


def _bf16(t: torch.Tensor) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise TypeError(f"the MI355X MoE kernels compute in bf16; got {t.dtype}")
    return t.contiguous()


_dense_tiles_cache = {}


def _dense_tiles(T: int, device):
    """Tile list of one dense group of T rows (group 0), for the router-backward GEMM."""
    key = (T, str(device))
    if key not in _dense_tiles_cache:
        n = (T + M_TILE - 1) // M_TILE
        t = torch.zeros(max(n, 1), 4, dtype=torch.int32)
        for i in range(n):
            t[i, 0], t[i, 1], t[i, 2], t[i, 3] = 0, i * M_TILE, min(T, (i + 1) * M_TILE), L.KIND_SHARED << 16
        _dense_tiles_cache[key] = (t.reshape(-1).to(device), torch.tensor([n], dtype=torch.int32, device=device),
                                   n, torch.tensor([L.KIND_SHARED << 16], dtype=torch.int32, device=device))
    return _dense_tiles_cache[key]


def _router_ext_weight(gate_w: torch.Tensor, sg_w: torch.Tensor | None, store: dict | None = None) -> PackedW:
    """The weight of the router-backward GEMM (dx += dlogits . W): router rows, then the shared-gate row, as one
    [E(+1), H] matrix in the transposed layout, its contraction dim padded to a multiple of 64 (R of the result)."""
    E, H = gate_w.shape
    Epad = (E + (1 if sg_w is not None else 0) + 63) // 64 * 64

    def build():
        if sg_w is None:
            pw = pack_bf16_t(gate_w)
        else:
            w = torch.empty(E + 1, H, dtype=torch.bfloat16, device=gate_w.device)
            w[:E] = gate_w
            w[E] = sg_w.reshape(-1)
            pw = pack_bf16_t(w)
        pw.R = Epad
        return pw

    return _cached("router_t", build, *((gate_w,) if sg_w is None else (gate_w, sg_w)), store=store)


_SIDE_STREAMS = {}
# Side streams: 0 = router backward, 1 = LoRA factor gradients, 2 = the forward's LoRA layouts. The default keeps
# 0 and 1: the layouts of both LoRA sets are one ~16 us launch, less than a fork and join of a graph costs there.
# SMEL_SIDE_STREAMS="0,1,2" (say) picks others; a fork that is off runs its launches on the main stream, in order.
_SIDE_ON = frozenset(int(v) for v in os.environ.get("SMEL_SIDE_STREAMS", "0,1").split(",") if v.strip())
# SMEL_BWD_ONE_SIDE=1 (default): the router backward and the LoRA factor gradients share one side stream, forked once
# after the down backward (after the gate_up LoRA projection when that is a launch of its own) and joined once before
# the dX reduce (each fork or join point of a replayed graph costs the main queue several µs); 0: each on its own
# stream, the router backward forked right after the down backward
_BWD_ONE_SIDE = os.environ.get("SMEL_BWD_ONE_SIDE", "1") == "1"
# SMEL_FWD_EXT_SIDE=1: with a fused shared expert that has a LoRA, the forward's LoRA layouts and the shared rows'
# gate_up LoRA projection (token order: no routing needed) run on side stream 2 beside the router and the dispatch;
# the main stream projects only the selected experts' rows after the dispatch. 0 (default): side stream 2 as
# SMEL_SIDE_STREAMS says, and one projection launch for all LoRA rows after the dispatch (the projection's time is
# its fixed latency, not its rows, so the split launch saves nothing on the main stream and the fork costs time)
_FWD_EXT_SIDE = os.environ.get("SMEL_FWD_EXT_SIDE", "0") == "1"
# SMEL_BWD_LORA_ROWS=1 (default): the gate_up backward's LoRA rows come from the down backward's epilogue as
# per-column-block partials (smel_gmm_bwd_lr), summed by the gate_up backward itself and, for the LoRA gradients, by
# smel_lora_rows_sum on the side stream: no smel_lora_ext launch between the two GEMMs; 0: that launch
_BWD_LORA_ROWS = os.environ.get("SMEL_BWD_LORA_ROWS", "1") == "1"
# SMEL_FWD_LORA_ROWS=1 (default): the down LoRA's rows come from the gate_up forward's epilogue as per-column-block
# partials (smel_gmm_fwd_lr), summed and stored by the down forward; 0: a smel_lora_ext launch over the gate_up
# output between the two GEMMs
_FWD_LORA_ROWS = os.environ.get("SMEL_FWD_LORA_ROWS", "1") == "1"
# SMEL_MERGE_SHORT=1 (default): the forward GEMMs take an int4 expert's last tile of at most 32 rows together with
# the full tile before it (one weight stream and dequant for up to 160 rows; banks in the fast dequant form), on the
# dispatch's merged tile list (the fused layer) or the merged count tiles (the frozen-experts path); 0: every tile of
# the list on its own
_MERGE_SHORT = os.environ.get("SMEL_MERGE_SHORT", "1") == "1"


def _side_stream(dev, i: int) -> torch.cuda.Stream:
    """Side stream i of a device (default priority), for launches that do not depend on the main stream's latest
    work: they overlap it, and the main stream waits for them before using their results (an event join, which a
    HIP graph capture records as a fork / join of the step graph)."""
    key = (str(dev), i)
    if key not in _SIDE_STREAMS:
        _SIDE_STREAMS[key] = torch.cuda.Stream(device=dev)
    return _SIDE_STREAMS[key]


class _Fork:
    """``with _Fork(dev, i) as s:`` launches on side stream i after the current stream's work so far; ``join()``
    makes the current (main) stream wait for everything launched there."""

    def __init__(self, dev, i: int, on: bool = None):
        self.main = torch.cuda.current_stream(dev)
        self.side = _side_stream(dev, i) if (i in _SIDE_ON if on is None else on) else self.main
        if self.side is not self.main:
            self.side.wait_stream(self.main)
        self._ctx = torch.cuda.stream(self.side)

    def __enter__(self):
        self._ctx.__enter__()
        return self.side

    def __exit__(self, *exc):
        return self._ctx.__exit__(*exc)

    def join(self):
        if self.side is not self.main:
            self.main.wait_stream(self.side)


class _LoRABufs:
    """bf16 K-extension layouts of one LoRA set (smel_lora_prep), built per call from the fp32 parameters. The
    gate_up side has ``planes`` 32-wide planes (a_gu, bt_gu: plane-major, one [n][32][K] matrix per plane; at_gu:
    [n][planes][H][32])."""

    def __init__(self, lora, n: int, H: int, I: int, device, planes: int = 1, prep: bool = True):
        self.scale = float(lora.scale)
        self.r = lora.r
        self.planes = planes
        self.H, self.I = H, I
        e = lambda *s: torch.empty(*s, dtype=torch.bfloat16, device=device)
        self.fwd_gu, self.fwd_dn = e(n, 2 * I, EXT), e(n, H, EXT)
        self.a_gu, self.a_dn = e(planes, n, EXT, H), e(n, EXT, I)
        self.bt_dn, self.bt_gu = e(n, EXT, H), e(planes, n, EXT, 2 * I)
        self.at_gu, self.at_dn = e(n, planes, H, EXT), e(n, I, EXT)
        self.factors = [getattr(lora, k).detach().float().contiguous() for k in
                        ("A_gate", "B_gate", "A_up", "B_up", "A_down", "B_down")]
        self.n = n
        if prep:
            _prep_sets([self])

    def lora_set(self) -> L.LoraSet:
        s = L.LoraSet(*[L.ptr(p) for p in self.factors], self.n, self.r)
        for k in ("fwd_gu", "fwd_dn", "a_gu", "a_dn", "bt_dn", "bt_gu", "at_gu", "at_dn"):
            setattr(s, k, L.ptr(getattr(self, k)))
        return s


def _prep_sets(bufs) -> None:
    """smel_lora_prep_sets: the bf16 layouts of one or two LoRA sets (same shapes and planes) in one launch."""
    bufs = [b for b in bufs if b is not None]
    if not bufs:
        return
    arr = (L.LoraSet * len(bufs))(*[b.lora_set() for b in bufs])
    b0 = bufs[0]
    L.call("smel_lora_prep_sets", arr, len(bufs), b0.planes, b0.H, b0.I, L.stream(), tag="smel_lora_prep")


_PLANE_MAJOR = ("a_gu", "bt_gu")   # layouts with a leading plane dimension (lora_ext operands)


def _lora_ext(tl, A, lda, a_rows, gather, order, TK, K, lb_ex, lb_sh, name: str, Kd: int, planes: int, M: int, dev,
              st, ext=None, row0: int = 0):
    """ext rows [M][32 * planes] of one direction: smel_lora_ext once per plane (``name`` = the layout the rows are
    projected on; the down side's layouts have one plane). ``tl`` = (tiles, n_tiles, max_tiles, gkind). ``ext`` = a
    buffer to fill instead of a new one, the tiles' row r going to its row row0 + r."""
    tiles, ntiles, maxt, gk = tl
    if ext is None:
        ext = torch.empty(M, EXT * planes, dtype=torch.bfloat16, device=dev)
    base = ext.data_ptr() + 2 * row0 * EXT * planes
    s_ex = lb_ex.scale if lb_ex is not None else 0.0
    s_sh = lb_sh.scale if lb_sh is not None else 0.0
    for c in range(planes):
        def w(lb):
            if lb is None:
                return None
            t = getattr(lb, name)
            return t[c] if name in _PLANE_MAJOR else t
        L.call("smel_lora_ext", L.ptr(tiles), L.ptr(ntiles), maxt, L.ptr(gk), L.ptr(A), lda, a_rows, gather,
               L.ptr(order), TK, K, L.ptr(w(lb_ex)), L.ptr(w(lb_sh)), Kd, s_ex, s_sh, base + 2 * EXT * c,
               EXT * planes, st)
    return ext


def _token_tiles(T: int, E: int, dev):
    """Rows [0, T) as M_TILE-row tiles of group E with the kind SMEL_KIND_SHARED in the entry's fourth field (the
    shared expert's rows, in token order), cached per shape: (tiles, n_tiles, max_tiles, gkind None)."""
    cache = _token_tiles.__dict__.setdefault("cache", {})
    key = (T, E, str(dev))
    if key not in cache:
        rows = [[E, r, min(r + M_TILE, T), L.KIND_SHARED << 16] for r in range(0, T, M_TILE)]
        t = torch.tensor(rows, dtype=torch.int32).reshape(-1).to(dev)
        cache[key] = (t, torch.tensor([len(rows)], dtype=torch.int32).to(dev), len(rows), None)
    return cache[key]


def _shared_lora_ext(x, K: int, E: int, bufs, dev):
    """The gate_up LoRA projection of the fused shared expert's rows [TK, TK + T) (x in token order, no routing
    needed) into a new ext buffer of all TK + T rows; the routed rows are filled after the dispatch."""
    lb_ex, lb_sh = bufs
    T, H = x.shape
    planes = (lb_ex or lb_sh).planes
    ext = torch.empty(T * K + T, EXT * planes, dtype=torch.bfloat16, device=dev)
    return _lora_ext(_token_tiles(T, E, dev), x, H, T, 0, None, 0, 1, None, lb_sh, "a_gu", H, planes, T, dev,
                     L.stream(), ext=ext, row0=T * K)


def _bwd_lora_rows(lb_ex, lb_sh, nblk: int, M: int, planes: int, dev):
    """smel_bwd_lora_rows for the down backward (producer) and the gate_up backward (consumer), with its fp32 partial
    buffer [M][nblk][planes][32]."""
    part = torch.empty(M, nblk, planes, EXT, dtype=torch.float32, device=dev)
    lr = L.BwdLoraRows(L.ptr(lb_ex.bt_gu) if lb_ex is not None else None,
                       L.ptr(lb_sh.bt_gu) if lb_sh is not None else None,
                       lb_ex.scale if lb_ex is not None else 0.0, lb_sh.scale if lb_sh is not None else 0.0,
                       lb_ex.n if lb_ex is not None else 0, planes, L.ptr(part), nblk)
    return lr, part


def _lora_rows_sum(tl, lr, lb_ex, lb_sh, M: int, planes: int, dev, st):
    """bf16 rows [M][32 planes] of the LoRA tiles from the partials of ``lr`` (for the LoRA gradients)."""
    tiles, ntiles, maxt, gk = tl
    ext = torch.empty(M, EXT * planes, dtype=torch.bfloat16, device=dev)
    L.call("smel_lora_rows_sum", L.ptr(tiles), L.ptr(ntiles), maxt, L.ptr(gk), int(lb_ex is not None),
           int(lb_sh is not None), lr.part, lr.parts, planes, L.ptr(ext), st, tag="smel_lora_rows")
    return ext


def _bank_wset(fz, which: str, t: bool = False) -> L.WSet:
    """smel_wset for the gate_up ('gu') or down ('dn') projection of a frozen bank (packed weights; t = the backward
    GEMM's transposed layout)."""
    w = L.WSet()
    if isinstance(fz, Int4Experts):
        d = fz.gu if which == "gu" else fz.dn
        qf, szf = fz.packed_t(which) if t else fz.packed(which)
        w.q4, w.sz4 = L.ptr(qf), L.ptr(szf)
        w.group = Int4Experts.group_of(d)
        w.flags = L.WSET_FAST_DQ if fz.fast_dq(which) else 0
        w.R, w.C = d["q"].shape[1], d["q"].shape[2] * 2
    else:
        pw = fz.packed_t(which) if t else fz.packed(which)
        w.wb = L.ptr(pw.t)
        w.group = 32
        w.R, w.C = pw.R, pw.C
    return w


def _wset(ex: LayerExperts, which: str, sel_w: PackedW | None, sh_w: PackedW | None, ext_sel, ext_sh,
          t: bool = False, planes: int = 1) -> L.WSet:
    """smel_wset for the gate_up ('gu') or down ('dn') projection of the layer (packed weights; t = transposed;
    planes = the gate_up LoRA K-extension's planes)."""
    w = _bank_wset(ex.frozen, which, t)
    w.wsel = L.ptr(sel_w.t) if sel_w is not None else None
    w.wsh = L.ptr(sh_w.t) if sh_w is not None else None
    w.ext_sel = L.ptr(ext_sel)
    w.ext_sh = L.ptr(ext_sh)
    if which == "gu" and planes == 2:
        w.flags |= L.WSET_EXT2
    return w


def _check_bank(ex):
    fz = ex.frozen if isinstance(ex, LayerExperts) else ex
    if isinstance(fz, Int4Experts):
        for d in (fz.gu, fz.dn):
            for k in ("q", "scale", "zero"):
                L.require_device(d[k])
                if not d[k].is_contiguous():
                    raise ValueError(f"int4 bank tensor {k} must be contiguous")
    else:
        for t in (fz.gate_up, fz.down):
            L.require_device(t)
            _bf16(t)


# ------------------------------------------------------------------------------------------------ shapes beyond the bf16 kernels


def _bf16_limit(H: int, ex=None, loras=(), mlp_I: int | None = None) -> str | None:
    """Why bf16 activations of these shapes cannot run on the bf16 kernels, or None: those take a hidden size that is
    a multiple of 64, intermediate sizes that are multiples of 32, int4 groups that are multiples of 32 and LoRA
    ranks up to 32. Such calls run on the fp32 kernels instead (bf16 in and out; every weight value the same, the
    int4 dequant rounded to bf16 as here), which the reference's shapes never need (its defaults are inside)."""
    if H % 64:
        return f"hidden {H} is not a multiple of 64"
    if ex is not None:
        fz = ex.frozen if isinstance(ex, LayerExperts) else ex
        I = (fz.dn["q"].shape[2] * 2) if isinstance(fz, Int4Experts) else fz.down.shape[2]
        if I % 32:
            return f"expert intermediate size {I} is not a multiple of 32"
        if isinstance(fz, Int4Experts) and any(Int4Experts.group_of(d) % 32 for d in (fz.gu, fz.dn)):
            return "int4 group not a multiple of 32"
    if mlp_I is not None and mlp_I % 32:
        return f"MLP intermediate size {mlp_I} is not a multiple of 32"
    r = max((m.r for m in loras if m is not None), default=0)
    if r > MAX_LORA_RANK:
        return f"LoRA rank {r} is above {MAX_LORA_RANK}"
    return None


def _f32_of(t: torch.Tensor, store: dict | None = None) -> torch.Tensor:
    """fp32 copy of a weight, reused while the source is unchanged (in ``store``, the layer's own, when given)."""
    return _cached("f32", lambda: t.float().contiguous(), t, store=store)


def _f32_W(W: dict, store: dict) -> dict:
    return {k: _f32_of(v, store) if torch.is_tensor(v) and v.is_floating_point() else v for k, v in W.items()}


def _f32_bank(fz, store: dict | None = None):
    """The frozen bank for the fp32 kernels: an int4 bank as is, dequantized and rounded to bf16 inside the GEMM (the
    values the bf16 kernels use); a bf16 bank as fp32 copies."""
    if isinstance(fz, Int4Experts):
        return _cached("f32_int4", lambda: Int4Experts(fz.gu, fz.dn, dtype=torch.bfloat16), fz.gu["q"], fz.dn["q"],
                       store=store)
    return _cached("f32_bank", lambda: BF16Experts(fz.gate_up.float().contiguous(), fz.down.float().contiguous()),
                   fz.gate_up, fz.down, store=store)


def _f32_experts(ex: LayerExperts, store: dict) -> LayerExperts:
    """The layer's experts for the fp32 kernels (selected experts as fp32 copies), kept in ``store``."""
    bank = _f32_bank(ex.frozen, store)
    if ex.sel_ids is None or not ex._slot:
        return _cached("f32_ex", lambda: LayerExperts(bank, group=ex.group, act=ex.act), *_bank_sources(ex.frozen),
                       store=store)
    return _cached("f32_ex", lambda: LayerExperts(bank, ex.sel_ids, ex.sel_gate_up.float().contiguous(),
                                                  ex.sel_down.float().contiguous(), ex.group, ex.act),
                   *_bank_sources(ex.frozen), ex.sel_gate_up, ex.sel_down, store=store)


def _bank_sources(fz):
    return (fz.gu["q"], fz.dn["q"]) if isinstance(fz, Int4Experts) else (fz.gate_up, fz.down)


# ------------------------------------------------------------------------------------------------ router


class _RouteFn(torch.autograd.Function):
    """route (smel/moe.py:162-167) with topv differentiable w.r.t. x through the router softmax."""

    @staticmethod
    def forward(ctx, x, gate_w, top_k):
        T, H = x.shape
        E = gate_w.shape[0]
        dev = x.device
        probs = torch.empty(T, E, dtype=torch.float32, device=dev)
        topv = torch.empty(T, top_k, dtype=torch.bfloat16, device=dev)
        topi = torch.empty(T, top_k, dtype=torch.int64, device=dev)
        topi32 = torch.empty(T, top_k, dtype=torch.int32, device=dev)
        lg = torch.empty(T, L.load().smel_route_ld(E, 0), dtype=torch.bfloat16, device=dev)
        L.call("smel_route", L.ptr(x), L.ptr(gate_w), None, T, H, E, top_k, L.ptr(probs), L.ptr(topv), None,
               L.ptr(topi), L.ptr(topi32), None, L.ptr(lg), L.stream())
        ctx.save_for_backward(probs, topi32, gate_w)
        ctx.mark_non_differentiable(probs, topi)
        return probs, topv, topi

    @staticmethod
    def backward(ctx, dprobs, dtopv, dtopi):
        probs, topi32, gate_w = ctx.saved_tensors
        T, E = probs.shape
        K = topi32.shape[1]
        dev = probs.device
        if dtopv is None:
            return None, None, None
        dwp = dtopv.float().contiguous().reshape(-1, 1)
        wr = _router_ext_weight(gate_w, None)
        Epad = wr.R
        dl = torch.empty(T, Epad, dtype=torch.bfloat16, device=dev)
        L.call("smel_route_bwd", L.ptr(dwp), 1, None, L.ptr(probs), L.ptr(topi32), None, None, 0, T, K, E, T * K,
               L.ptr(dl), Epad, None, None, L.stream())
        dx = _router_dx(dl, wr, T)
        return dx, None, None


def _router_dx(dl: torch.Tensor, wr: PackedW, T: int, dx: torch.Tensor | None = None) -> torch.Tensor:
    H = wr.C
    tiles, ntiles, maxt, gk = _dense_tiles(T, dl.device)
    if dx is None:
        dx = torch.empty(T, H, dtype=torch.bfloat16, device=dl.device)
    w = L.WSet()
    w.wsh = L.ptr(wr.t)
    w.R, w.C, w.group = wr.R, H, 32
    L.call("smel_gmm_bwd", ctypes.byref(w), L.ptr(gk), L.ptr(tiles), L.ptr(ntiles), maxt, L.ptr(dl), dl.shape[1], T, 0,
           None, 0, 1, None, 0, 0, None, None, None, L.ptr(dx), H, None, L.stream(), tag="gemm_router_bwd")
    return dx


def route(x2d, gate_w, top_k):
    """smel/moe.py:162-167 -> (probs fp32 [T,E], topv [T,K] renormalised in the logits' dtype, topi int64 [T,K]).
    bf16 or fp32 activations (the fp32 path: every product an fp32 MFMA)."""
    L.require_device(x2d, gate_w)
    if x2d.dtype == torch.float32:
        return F32.RouteFn.apply(F32.f32(x2d), F32.f32(gate_w, "gate_w"), int(top_k))
    if _bf16_limit(x2d.shape[-1]) is not None:
        probs, topv, topi = F32.RouteFn.apply(x2d.float(), _f32_of(_bf16(gate_w)), int(top_k))
        return probs, topv.to(x2d.dtype), topi
    return _RouteFn.apply(_bf16(x2d), _bf16(gate_w), int(top_k))


class _RouteGemma4Fn(torch.autograd.Function):
    """route_gemma4 (smel/moe.py:170-180): topv differentiable w.r.t. h through the per-expert scale, the renorm, the
    softmax, the router GEMM and the weightless RMSNorm."""

    @staticmethod
    def forward(ctx, h, scale, proj, pes, top_k, eps):
        T, H = h.shape
        E = proj.shape[0]
        dev = h.device
        probs = torch.empty(T, E, dtype=torch.float32, device=dev)
        topv = torch.empty(T, top_k, dtype=torch.float32, device=dev)
        topi = torch.empty(T, top_k, dtype=torch.int64, device=dev)
        topi32 = torch.empty(T, top_k, dtype=torch.int32, device=dev)
        xn = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
        rstd = torch.empty(T, dtype=torch.float32, device=dev)
        lg = torch.empty(T, L.load().smel_route_ld(E, 0), dtype=torch.bfloat16, device=dev)
        L.call("smel_route_gemma4", L.ptr(h), L.ptr(scale), L.ptr(proj), L.ptr(pes), T, H, E, top_k, eps,
               L.ptr(probs), L.ptr(topv), L.ptr(topi), L.ptr(topi32), L.ptr(xn), L.ptr(rstd), L.ptr(lg), L.stream())
        ctx.save_for_backward(h, scale, proj, pes, probs, topi32, rstd)
        ctx.mark_non_differentiable(probs, topi)
        return probs, topv, topi

    @staticmethod
    def backward(ctx, dprobs, dtopv, dtopi):
        if dtopv is None:
            return None, None, None, None, None, None
        h, scale, proj, pes, probs, topi32, rstd = ctx.saved_tensors
        T, H = h.shape
        E, K = probs.shape[1], topi32.shape[1]
        dev = h.device
        wr = _router_ext_weight(proj, None)
        dl = torch.empty(T, wr.R, dtype=torch.bfloat16, device=dev)
        dw = dtopv.float().contiguous()
        L.call("smel_route_bwd", L.ptr(dw), 1, None, L.ptr(probs), L.ptr(topi32), None, None, 0, T, K, E, T * K,
               L.ptr(dl), wr.R, None, L.ptr(pes), L.stream())
        dxn = _router_dx(dl, wr, T)
        dh = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
        L.call("smel_route_gemma4_prenorm_bwd", L.ptr(h), L.ptr(scale), L.ptr(rstd), L.ptr(dxn), T, H, L.ptr(dh),
               L.stream())
        return dh, None, None, None, None, None


def route_gemma4(h, W, top_k, eps):
    """Gemma 4 router on the residual stream (smel/moe.py:170-180) -> (probs fp32 [T,E], topv fp32 [T,K] =
    renormalised top-k x per_expert_scale, topi int64 [T,K]): weightless RMSNorm, x router.scale x H^-0.5, logits,
    softmax, top-k, renorm, scale, as HIP kernels (differentiable w.r.t. h)."""
    L.require_device(h)
    if h.dtype == torch.bfloat16 and _bf16_limit(h.shape[-1]) is not None:
        return F32.RouteGemma4Fn.apply(h.float(), _f32_of(_bf16(W["router.scale"])).reshape(-1),
                                       _f32_of(_bf16(W["router.proj.weight"])),
                                       _f32_of(_bf16(W["router.per_expert_scale"])).reshape(-1), int(top_k), float(eps))
    if h.dtype == torch.float32:
        return F32.RouteGemma4Fn.apply(F32.f32(h), F32.f32(W["router.scale"], "router.scale").reshape(-1),
                                       F32.f32(W["router.proj.weight"], "router.proj.weight"),
                                       F32.f32(W["router.per_expert_scale"], "router.per_expert_scale").reshape(-1),
                                       int(top_k), float(eps))
    return _RouteGemma4Fn.apply(_bf16(h), _bf16(W["router.scale"]).reshape(-1), _bf16(W["router.proj.weight"]),
                                _bf16(W["router.per_expert_scale"]).reshape(-1), int(top_k), float(eps))


# ------------------------------------------------------------------------------------------------ fused layer


class _Ctx:
    pass


def _lora_groups(ex: LayerExperts, with_shared: bool, n_sel_lora: int, device):
    """Group ids that carry LoRA (selected experts, then the shared expert as group E), cached on the layer so that
    a step makes no host-to-device copy (and can be captured in a HIP graph)."""
    cache = ex.__dict__.setdefault("_lora_groups", {})
    key = (with_shared, n_sel_lora, str(device))
    if key not in cache:
        ids = [int(e) for e in ex.sel_ids.tolist()][:n_sel_lora] if (ex.sel_ids is not None and n_sel_lora) else []
        if with_shared:
            ids.append(ex.E)
        cache[key] = torch.tensor(ids, dtype=torch.int32, device=device)
    return cache[key]


def _expert_I(ex: LayerExperts) -> int:
    return (ex.frozen.dn["q"].shape[2] * 2) if isinstance(ex.frozen, Int4Experts) else ex.frozen.down.shape[2]


def _prep_lora(ex: LayerExperts, lora_ex, lora_sh, with_shared: bool, H: int, dev):
    """The bf16 LoRA layouts of the selected experts and the shared MLP (lora_prep launches on the current stream),
    with the gate_up planes both sets need."""
    I = _expert_I(ex)
    has_sel = ex.sel_ids is not None and len(ex._slot)
    use_ex = lora_ex if (lora_ex is not None and has_sel) else None
    use_sh = lora_sh if (lora_sh is not None and with_shared) else None
    planes = _lora_planes(use_ex, use_sh)
    lb_ex = _LoRABufs(use_ex, len(ex._slot), H, I, dev, planes, prep=False) if use_ex is not None else None
    lb_sh = _LoRABufs(use_sh, 1, H, I, dev, planes, prep=False) if use_sh is not None else None
    _prep_sets([lb_ex, lb_sh])   # both sets in one launch
    return lb_ex, lb_sh


def _forward_pipeline(x, ex: LayerExperts, K: int, topv, topi_ids, ids_i64: bool, shared, lora_ex, lora_sh,
                      need_grad: bool, c: _Ctx, prep=None, shared_rows=None, counted_ws=None, ext_pre=None):
    """Dispatch + expert GEMMs + combine. ``shared`` = (gate_up, down, sgate fp32 [T], gate_up^T, down^T) or None
    (packed forward and transposed layouts of the shared expert's [2I,H] / [H,I] weights). ``prep`` = (_Fork,
    (lb_ex, lb_sh)) when the LoRA layouts were launched on a side stream (joined before their first use).
    ``shared_rows`` = (sgate fp32 [T], y_shared bf16 [T, H]) adds a shared expert computed elsewhere (one whose
    intermediate size differs from the experts') to the combine. ``counted_ws`` = the dispatch workspace that
    smel_route_counted filled for these ids (the dispatch then skips its histogram launch). ``ext_pre`` = the gate_up
    LoRA rows with the shared rows already projected (_shared_lora_ext, on the fork of ``prep``)."""
    T, H = x.shape
    E = ex.E
    dev = x.device
    st = L.stream()
    TK = T * K
    rows_sh = T if shared is not None else 0
    M = TK + rows_sh
    maxt = L.load().smel_dispatch_max_tiles(TK, E, rows_sh, M_TILE)
    i32 = lambda *s: torch.empty(*s, dtype=torch.int32, device=dev)
    counts, offsets, order, inv = i32(E), i32(E + 1), i32(max(TK, 1)), i32(max(TK, 1))
    tiles, tiles_g, ntiles, err = i32(maxt * 4), i32(maxt * 4), i32(1), i32(1)
    # the gate_up forward's merged tile list: an int4 expert's last tile of <= 32 rows joins its full tile
    fz = ex.frozen
    merge = _MERGE_SHORT and isinstance(fz, Int4Experts) and H % 64 == 0 and fz.fast_dq("gu")
    tiles_m, ntiles_m = (i32(maxt * 4), i32(1)) if merge else (None, None)
    dws = counted_ws if counted_ws is not None else i32(max(1, L.load().smel_dispatch_ws_size(TK, E)))
    if prep is None:   # LoRA layouts on a side stream, overlapping the dispatch
        fork = _Fork(dev, 2)
        with fork:
            bufs = _prep_lora(ex, lora_ex, lora_sh, shared is not None, H, dev)
        prep = (fork, bufs)
    gk_groups = ex.gkind(shared is not None, dev)
    L.call("smel_dispatch_counted" if counted_ws is not None else "smel_dispatch", L.ptr(topi_ids), int(ids_i64), T, K,
           E, rows_sh, M_TILE, L.ptr(gk_groups), L.ptr(counts), L.ptr(offsets), L.ptr(order), L.ptr(inv), L.ptr(tiles),
           L.ptr(tiles_g), L.ptr(ntiles), L.ptr(err), M_MERGED if merge else 0, L.ptr(tiles_m), L.ptr(ntiles_m),
           L.ptr(dws), st, tag="smel_dispatch")
    gk = None   # the tile list carries each tile's group kind
    sel_gu = sel_dn = None
    if ex.sel_ids is not None and len(ex._slot):
        sel_gu, sel_dn = ex.packed_sel()
    I = _expert_I(ex)
    sh_gu = sh_dn = sgate = sh_gu_t = sh_dn_t = None
    if shared is not None:
        sh_gu, sh_dn, sgate, sh_gu_t, sh_dn_t = shared
    fork, (lb_ex, lb_sh) = prep
    fork.join()
    any_lora = lb_ex is not None or lb_sh is not None
    planes = (lb_ex or lb_sh).planes if any_lora else 1
    g = lambda b, n: getattr(b, n) if b is not None else None
    bf = lambda *s: torch.empty(*s, dtype=torch.bfloat16, device=dev)
    tl = (tiles, ntiles, maxt, gk)
    ext_gu = ext_dn = None
    if any_lora and ext_pre is not None:   # the shared rows are done: the selected experts' rows only
        ext_gu = ext_pre
        if lb_ex is not None:
            _lora_ext(tl, x, H, T, 1, order, TK, K, lb_ex, None, "a_gu", H, planes, M, dev, st, ext=ext_gu)
    elif any_lora:
        ext_gu = _lora_ext(tl, x, H, T, 1, order, TK, K, lb_ex, lb_sh, "a_gu", H, planes, M, dev, st)
    actb = bf(M, I)
    hsave = bf(M, 2 * I) if need_grad else None
    # the gate_up forward takes the merged list (tile t on XCD t % 8, the merged tiles first) or else the tiles in
    # group order, a chunk per XCD (an expert's tiles share its weights in L2); the down GEMMs the long-tiles-first
    # order (short tiles fill the last round)
    w_gu = _wset(ex, "gu", sel_gu, sh_gu, g(lb_ex, "fwd_gu"), g(lb_sh, "fwd_gu"), planes=planes)
    w_gu.flags |= L.WSET_MERGED_LIST if merge else L.WSET_XCD_CHUNK
    # the down LoRA's rows come from the gate_up epilogue (per-column-block partials of h A_dn^T), summed and stored
    # by the down GEMM: no separate projection launch
    lr = None
    if any_lora and _FWD_LORA_ROWS:
        parts = int(L.load().smel_gmm_fwd_nblocks(2 * I, 1))
        xpart = torch.empty(M, parts, EXT, dtype=torch.float32, device=dev)
        ext_dn = bf(M, EXT)
        lr = L.FwdLoraRows(L.ptr(g(lb_ex, "a_dn")), L.ptr(g(lb_sh, "a_dn")), lb_ex.scale if lb_ex is not None else 0.0,
                           lb_sh.scale if lb_sh is not None else 0.0, L.ptr(xpart), parts, L.ptr(ext_dn))
    L.call("smel_gmm_fwd_lr", ctypes.byref(w_gu), L.ptr(gk), L.ptr(tiles_m if merge else tiles_g),
           L.ptr(ntiles_m if merge else ntiles), maxt, L.ptr(x), H, T, 1,
           L.ptr(order), TK, K, L.ptr(ext_gu), 1, _ACT[ex.act], L.ptr(actb), I, L.ptr(hsave),
           ctypes.byref(lr) if lr is not None else None, st, tag="gemm_gu_fwd")
    if any_lora and lr is None:   # the down LoRA's rows as a projection launch of the gate_up output
        ext_dn = _lora_ext(tl, actb, I, M, 0, order, TK, K, lb_ex, lb_sh, "a_dn", I, 1, M, dev, st)
    Y = bf(M, H)
    w_dn = _wset(ex, "dn", sel_dn, sh_dn, g(lb_ex, "fwd_dn"), g(lb_sh, "fwd_dn"))
    # the down forward on the same merged list when its bank is in the fast form too (and I a multiple of 64)
    merge_dn = merge and I % 64 == 0 and fz.fast_dq("dn")
    if merge_dn:
        w_dn.flags |= L.WSET_MERGED_LIST
    L.call("smel_gmm_fwd_lr", ctypes.byref(w_dn), L.ptr(gk), L.ptr(tiles_m if merge_dn else tiles),
           L.ptr(ntiles_m if merge_dn else ntiles), maxt, L.ptr(actb), I, M, 0,
           L.ptr(order), TK, K, L.ptr(ext_dn) if lr is None else None, 0, _ACT[ex.act], L.ptr(Y), H, None,
           ctypes.byref(lr) if lr is not None else None, st, tag="gemm_dn_fwd")
    out = bf(T, H)
    ysh = None
    if shared_rows is not None:
        sgate, ysh = shared_rows
    L.call("smel_combine", L.ptr(Y), L.ptr(topv), L.ptr(inv), L.ptr(sgate), L.ptr(ysh), T, K, H, L.ptr(out), st)
    # everything the backward needs
    c.T, c.H, c.I, c.E, c.K, c.TK, c.M, c.maxt = T, H, I, E, K, TK, M, maxt
    c.ex, c.shared_w = ex, (sh_gu_t, sh_dn_t) if shared is not None else None
    sel_t = ex.packed_sel_t() if (need_grad and sel_gu is not None) else None
    c.tensors = dict(x=x, topv=topv, sgate=sgate, counts=counts, offsets=offsets, order=order, inv=inv, tiles=tiles,
                     tiles_g=tiles_g, ntiles=ntiles, err=err, gk=gk, act=actb, hsave=hsave, ext_gu=ext_gu,
                     ext_dn=ext_dn, sel_gu=sel_t[0] if sel_t else None, sel_dn=sel_t[1] if sel_t else None)
    c.lb_ex, c.lb_sh = lb_ex, lb_sh
    c.lora_ex, c.lora_sh = lora_ex, lora_sh
    return out


def _backward_pipeline(c: _Ctx, dout: torch.Tensor, router=None, shared_split=None):
    """Returns (dx_experts_plus_router, dtopv or None, {lora_param_name: grad}). ``router`` = (probs, topi32, wr) for
    the fused layer (router + shared gate backward folded into the dX reduce). ``shared_split`` = (dwp_sh, nblk_sh,
    dx_sh) of a shared expert that ran as its own GEMMs: its row-weight partials (for the shared gate's gradient) and
    its dX rows."""
    t = c.tensors
    T, H, I, E, K, TK, M, maxt = c.T, c.H, c.I, c.E, c.K, c.TK, c.M, c.maxt
    dev = dout.device
    st = L.stream()
    ex = c.ex
    dout = _bf16(dout)
    lb_ex, lb_sh = c.lb_ex, c.lb_sh
    g = lambda b, n: getattr(b, n) if b is not None else None
    any_lora = lb_ex is not None or lb_sh is not None
    planes = (lb_ex or lb_sh).planes if any_lora else 1
    bf = lambda *s: torch.empty(*s, dtype=torch.bfloat16, device=dev)
    sh_gu, sh_dn = c.shared_w if c.shared_w is not None else (None, None)
    order, tiles, ntiles, gk = t["order"], t["tiles"], t["ntiles"], t["gk"]
    tl = (tiles, ntiles, maxt, gk)
    # (1) LoRA down-projection of dout for the down backward: DB = s dout B_d (not yet scaled by the row weight)
    ext_db = None
    if any_lora:
        ext_db = _lora_ext(tl, dout, H, T, 1, order, TK, K, lb_ex, lb_sh, "bt_dn", H, 1, M, dev, st)
    # (2) down backward + SiLU-gate backward + d(row weight) partials
    nblk = L.load().smel_gmm_bwd_nblocks(I)
    dh = bf(M, 2 * I)
    dwp = torch.empty(M, nblk, dtype=torch.float32, device=dev)
    w_dn = _wset(ex, "dn", t["sel_dn"], sh_dn, g(lb_ex, "at_dn"), g(lb_sh, "at_dn"), t=True)
    # with the LoRA rows from this GEMM's epilogue: DXA = s [dg B_g, du B_u] as per-column-block partials
    lrows = _bwd_lora_rows(lb_ex, lb_sh, nblk, M, planes, dev) if any_lora and _BWD_LORA_ROWS else None
    lr = ctypes.byref(lrows[0]) if lrows is not None else None
    L.call("smel_gmm_bwd_lr", ctypes.byref(w_dn), L.ptr(gk), L.ptr(tiles), L.ptr(ntiles), maxt, L.ptr(dout), H, T, 1,
           L.ptr(order), TK, K, L.ptr(ext_db), 1, _ACT[ex.act], L.ptr(t["hsave"]), L.ptr(t["topv"]), L.ptr(t["sgate"]),
           L.ptr(dh), 2 * I, L.ptr(dwp), lr, st, tag="gemm_dn_bwd")
    # (3) LoRA B^T projection of dh for the gate_up backward: DXA = s [dg B_g, du B_u] (without the partials)
    ext_dxa = None
    if any_lora and _BWD_ONE_SIDE and lrows is None:
        ext_dxa = _lora_ext(tl, dh, 2 * I, M, 0, order, TK, K, lb_ex, lb_sh, "bt_gu", 2 * I, planes, M, dev, st)
    # (5, side stream 0) router backward (fused layer) or d topv (routed_experts): needs only dwp, so it overlaps
    # steps (3) and (4)
    dxr = None
    dtopv = None
    side_r = _Fork(dev, 0)
    if router is not None:
        probs, topi32, wr = router
        Epad = wr.R
        dl = bf(T, Epad)
        dxr = bf(T, H)
        with side_r:
            dwp_sh, nblk_sh = (shared_split[0], shared_split[1]) if shared_split is not None else (None, 0)
            L.call("smel_route_bwd", L.ptr(dwp), nblk, L.ptr(t["inv"]), L.ptr(probs), L.ptr(topi32),
                   L.ptr(t["sgate"]), L.ptr(dwp_sh), nblk_sh, T, K, E, TK, L.ptr(dl), Epad, None, None, L.stream())
            _router_dx(dl, wr, T, dxr)
    else:
        dtopv = torch.empty(T, K, dtype=torch.float32, device=dev)
        with side_r:
            L.call("smel_dtopv", L.ptr(dwp), nblk, L.ptr(t["inv"]), TK, L.ptr(dtopv), L.stream())
    if any_lora and not _BWD_ONE_SIDE and lrows is None:
        ext_dxa = _lora_ext(tl, dh, 2 * I, M, 0, order, TK, K, lb_ex, lb_sh, "bt_gu", 2 * I, planes, M, dev, st)
    # (6, side stream 1, or after the router backward on stream 0) LoRA factor gradients: one launch for the four
    # products, written into parameter-shaped fp32 tensors; every operand is ready here, so it overlaps the gate_up
    # backward
    grads = {}
    side_w = None
    if any_lora:
        n_sel = len(ex._slot) if lb_ex is not None else 0
        groups = _lora_groups(ex, lb_sh is not None, n_sel, dev)
        sets = ((c.lora_ex if lb_ex is not None else None), (c.lora_sh if lb_sh is not None else None))
        gx, gs = (_alloc_lora_grads(m, dev) for m in sets)
        if lrows is not None:
            ext_dxa = torch.empty(M, EXT * planes, dtype=torch.bfloat16, device=dev)   # filled on the side stream
        jobs, nj = _wgrad_jobs(H, I, (gx, gs), sets, (ext_dxa, t["x"], T, 1, 0), (t["ext_gu"], dh, M, 0, 0),
                               (ext_db, t["act"], M, 0, 1), (t["ext_dn"], dout, T, 1, 1), planes)
        # rows of all LoRA groups: a token routes at most min(K, n_sel) slots to selected experts, + the shared rows
        max_rows = (min(K, n_sel) * T if lb_ex is not None else 0) + (T if lb_sh is not None else 0)
        ws = _wgrad_ws(jobs, nj, groups.numel(), max_rows, dev)
        side_w = side_r if _BWD_ONE_SIDE else _Fork(dev, 1)
        with side_w:
            if lrows is not None:
                L.call("smel_lora_rows_sum", L.ptr(tiles), L.ptr(ntiles), maxt, L.ptr(gk), int(lb_ex is not None),
                       int(lb_sh is not None), L.ptr(lrows[1]), nblk, planes, L.ptr(ext_dxa), L.stream(),
                       tag="smel_lora_rows")
            L.call("smel_lora_wgrad", jobs, nj, L.ptr(groups), groups.numel(), n_sel, L.ptr(t["offsets"]), E, T, TK,
                   K, L.ptr(order), L.ptr(t["topv"]), L.ptr(t["sgate"]), max_rows, L.ptr(ws), ws.numel(), L.stream(),
                   tag="lora_wgrad")
        if gx is not None:
            grads["ex"] = gx
        if gs is not None:
            grads["sh"] = gs
    # (4) gate_up backward: per-slot dx rows
    dxs = bf(M, H)
    w_gu = _wset(ex, "gu", t["sel_gu"], sh_gu, g(lb_ex, "at_gu"), g(lb_sh, "at_gu"), t=True, planes=planes)
    w_gu.flags |= L.WSET_XCD_CHUNK
    L.call("smel_gmm_bwd_lr", ctypes.byref(w_gu), L.ptr(gk), L.ptr(t["tiles_g"]), L.ptr(ntiles), maxt, L.ptr(dh),
           2 * I, M, 0, L.ptr(order), TK, K, None if lrows is not None else L.ptr(ext_dxa), 0, _ACT[ex.act], None, None,
           None, L.ptr(dxs), H, None, lr, st, tag="gemm_gu_bwd")
    side_r.join()
    dx = bf(T, H)
    dxsh = shared_split[2] if shared_split is not None else None
    L.call("smel_dx_reduce", L.ptr(dxs), L.ptr(dxr), L.ptr(t["inv"]), int(t["sgate"] is not None), L.ptr(dxsh), T,
           K, H, L.ptr(dx), st)
    if side_w is not None and side_w is not side_r:
        side_w.join()
    return dx, dtopv, grads


_LORA_NAMES = ("A_gate", "B_gate", "A_up", "B_up", "A_down", "B_down")


def _lora_leaves(lora):
    return [getattr(lora, n) for n in _LORA_NAMES] if lora is not None else []


def _shape_grads(grads: dict, tag: str, lora, squeeze: bool = False):
    """The parameter-shaped LoRA gradients of one set (None where a parameter needs none)."""
    if lora is None:
        return []
    if tag not in grads:
        return [None] * 6
    return [grads[tag].get(n) for n in _LORA_NAMES]


def _alloc_lora_grads(lora, device):
    """fp32 gradient tensors shaped like the LoRA parameters that require a gradient (each element is written by the
    weight-gradient kernel), or None without the set."""
    if lora is None:
        return None
    return {n: torch.empty(getattr(lora, n).shape, dtype=torch.float32, device=device)
            for n in _LORA_NAMES if getattr(lora, n).requires_grad}


def _wgrad_ws(jobs, n_jobs: int, n_lora: int, max_rows: int, device) -> torch.Tensor:
    """fp32 workspace of smel_lora_wgrad (partial tiles of the groups longer than one 512-row chunk)."""
    n = L.load().smel_lora_wgrad_ws_floats(jobs, n_jobs, n_lora, max_rows)
    return torch.empty(max(n, 1), dtype=torch.float32, device=device)


def _wgrad_jobs(H, I, grads, sets, j_agu, j_bgu, j_adn, j_bdn, planes: int = 1):
    """The smel_wg_job list of a backward: dA and dB of gate/up, dA and dB of down. Each j_* = (L rows, Rm, Rm rows,
    r_gather, use_w). Destinations: class 0 = the selected experts' ExpertsLoRA (slot = its index), class 1 = the
    shared MLPLoRA. With one gate_up plane a gate/up product is one job whose result splits in two halves (ranks
    0..15 / 16..31; the B factors' columns 0..I-1 / I..2I-1); with two planes it is one job per plane (L = that
    plane's 32 columns of the 64-wide ext rows; the up B job reads the up half of dh only). Returns (jobs, count)."""
    gate_up = []   # (L byte offset, ldl, Rm byte offset, Q, [(half, param, p0, q0, nq, col_major)])
    if planes == 1:
        gate_up.append((j_agu, 0, EXT, 0, H, [(0, "A_gate", 0, 0, H, False), (1, "A_up", EXT // 2, 0, H, False)]))
        gate_up.append((j_bgu, 0, EXT, 0, 2 * I,
                        [(0, "B_gate", 0, 0, I, True), (1, "B_up", EXT // 2, I, I, True)]))
    else:
        w = 2 * EXT
        gate_up.append((j_agu, 0, w, 0, H, [(0, "A_gate", 0, 0, H, False)]))
        gate_up.append((j_agu, 2 * EXT, w, 0, H, [(0, "A_up", 0, 0, H, False)]))
        gate_up.append((j_bgu, 0, w, 0, I, [(0, "B_gate", 0, 0, I, True)]))
        gate_up.append((j_bgu, 2 * EXT, w, 2 * I, I, [(0, "B_up", 0, 0, I, True)]))
    specs = gate_up + [(j_adn, 0, EXT, 0, I, [(0, "A_down", 0, 0, I, False)]),
                       (j_bdn, 0, EXT, 0, H, [(0, "B_down", 0, 0, H, True)])]
    jobs = (L.WgJob * len(specs))()
    for J, ((Lb, Rm, rows, gather, use_w), l_off, ldl, r_off, Q, dests) in zip(jobs, specs):
        J.L, J.Rm = Lb.data_ptr() + l_off, Rm.data_ptr() + r_off
        J.ldl, J.ldr, J.r_rows, J.r_gather, J.use_w, J.Q = ldl, Rm.shape[1], rows, gather, use_w, Q
        for cls in range(2):
            g, m = grads[cls], sets[cls]
            if g is None:
                continue
            lead = 1 if cls == 0 else 0
            for h, name, p0, q0, nq, col_major in dests:
                t = g.get(name)
                if t is None:
                    continue
                d = J.dest[cls][h]
                d.ptr = L.ptr(t)
                d.s_idx = t.stride(0) if lead else 0
                # A factors [.., r, Q] (p rows, q contiguous); B factors [.., Q, r] (q rows, p contiguous)
                d.s_p, d.s_q = (1, t.stride(lead)) if col_major else (t.stride(lead), 1)
                d.p0, d.np, d.q0, d.nq = p0, m.r, q0, nq
    return jobs, len(specs)


class _MoELayerFn(torch.autograd.Function):
    """The fused MoE layer (moe_forward): router + routed experts + shared expert, one forward and one backward. A
    shared expert whose intermediate size equals the experts' is group E of the expert GEMMs; another size runs as its
    own dense-group GEMMs (row weight = the shared gate) and joins in the combine and the dX reduce."""

    @staticmethod
    def forward(ctx, x, plan, stats, *leaves):
        T, H = x.shape
        E, K = plan["ex"].E, plan["top_k"]
        dev = x.device
        has_sh = plan["shared"] is not None
        split = has_sh and plan["split_shared"]
        fuse = has_sh and not split
        probs = torch.empty(T, E, dtype=torch.float32, device=dev)
        topv = torch.empty(T, K, dtype=torch.bfloat16, device=dev)
        topv32 = torch.empty(T, K, dtype=torch.float32, device=dev)   # fp32 of topv: the combine weight
        topi = torch.empty(T, K, dtype=torch.int64, device=dev)
        topi32 = torch.empty(T, K, dtype=torch.int32, device=dev)
        sgate = torch.empty(T, dtype=torch.float32, device=dev) if has_sh else None
        sgw = plan["shared"][2] if has_sh else None
        lg = torch.empty(T, L.load().smel_route_ld(E, int(has_sh)), dtype=torch.bfloat16, device=dev)
        # LoRA layouts (and the shared rows' LoRA projection) overlap the router and the dispatch
        side_ext = _FWD_EXT_SIDE and fuse and plan["lora_sh"] is not None
        fork = _Fork(dev, 2, on=True if side_ext else None)
        ext_pre = None
        with fork:
            bufs = _prep_lora(plan["ex"], plan["lora_ex"], plan["lora_sh"] if fuse else None, fuse, H, dev)
            if side_ext and bufs[1] is not None:
                ext_pre = _shared_lora_ext(x, K, E, bufs, dev)
        # the router also counts the dispatch's per-block histograms of its picks into the dispatch workspace
        dws = torch.empty(max(1, L.load().smel_dispatch_ws_size(T * K, E)), dtype=torch.int32, device=dev)
        L.call("smel_route_counted", L.ptr(x), L.ptr(plan["gate_w"]), L.ptr(sgw), T, H, E, K, L.ptr(probs),
               L.ptr(topv), L.ptr(topv32), L.ptr(topi), L.ptr(topi32), L.ptr(sgate), L.ptr(lg), L.ptr(dws), L.stream(),
               tag="smel_route")
        if stats is not None:
            stats(probs, topv, topi)
        c = _Ctx()
        shared = (plan["shared"][0], plan["shared"][1], sgate, plan["shared"][4], plan["shared"][5]) if fuse else None
        shared_rows = None
        if split:
            pgu, pdn, _, Is, pgu_t, pdn_t = plan["shared"]
            lsh = plan["lora_sh"]
            lb_sh = _LoRABufs(lsh, 1, H, Is, dev, _lora_planes(lsh)) if lsh is not None else None
            ysh, sv = _dense_mlp_fwd(x, pgu, pdn, lb_sh, "silu", tag="gemm_shared")
            shared_rows = (sgate, ysh)
            c.split = (sv, pgu_t, pdn_t, lsh, sgate)
        out = _forward_pipeline(x, plan["ex"], K, topv32, topi32, False, shared, plan["lora_ex"],
                                plan["lora_sh"] if fuse else None, plan["need_grad"], c, prep=(fork, bufs),
                                shared_rows=shared_rows, counted_ws=dws, ext_pre=ext_pre)
        if plan["need_grad"]:
            c.router = (probs, topi32, _router_ext_weight(plan["gate_w"], sgw, plan["store"]))
            c.plan_lora_sh = plan["lora_sh"]
            ctx.c = c
        return out

    @staticmethod
    def backward(ctx, dout):
        c = ctx.c
        split = getattr(c, "split", None)
        shared_split = None
        grads_sh = None
        if split is not None:
            sv, pgu_t, pdn_t, lsh, sgate = split
            dx_sh, grads_sh, dwp_sh, nblk_sh = _dense_mlp_bwd(sv, dout, pgu_t, pdn_t, lsh, "silu", sgate,
                                                              tag="gemm_shared")
            shared_split = (dwp_sh, nblk_sh, dx_sh)
        dx, _, grads = _backward_pipeline(c, dout, router=c.router, shared_split=shared_split)
        if grads_sh is not None:
            grads["sh"] = grads_sh
        g = _shape_grads(grads, "ex", c.lora_ex) + _shape_grads(grads, "sh", c.plan_lora_sh)
        ctx.c = None
        return (dx, None, None, *g)


class _RoutedFn(torch.autograd.Function):
    """routed_experts (smel/moe.py:214-252) with given routing: differentiable w.r.t. x2d, topv and expert LoRA."""

    @staticmethod
    def forward(ctx, x, topv, topi, ex, lora, *leaves):
        c = _Ctx()
        K = topi.shape[1]
        tv = topv.detach().float().contiguous()   # fp32 combine weights: the reference's topv.float() (:252)
        need = ctx.needs_input_grad[0] or ctx.needs_input_grad[1] or any(ctx.needs_input_grad[5:])
        out = _forward_pipeline(x, ex, K, tv, topi.contiguous(), topi.dtype == torch.int64, None, lora, None, need, c)
        _ID_CHECK.record(c.tensors["err"])
        if need:
            ctx.c = c
        ctx.topv_dtype = topv.dtype
        return out

    @staticmethod
    def backward(ctx, dout):
        c = ctx.c
        dx, dtopv, grads = _backward_pipeline(c, dout, router=None)
        g = _shape_grads(grads, "ex", c.lora_ex)
        ctx.c = None
        return (dx, dtopv.to(ctx.topv_dtype), None, None, None, *g)


class _DeferredIdCheck:
    """Expert ids handed in by a caller must lie in [0, E) (the reference's bincount / indexing, smel/moe.py:216-223,
    fails otherwise, on the GPU asynchronously). The dispatch kernel checks them itself: it drops a slot whose id is
    out of range (inv = -1; the combine, the dX reduce and the d(topv) reduction read it as a zero row, so outputs and
    gradients stay defined) and sets bit 0 of its error word. Each eager call copies that word into pinned host memory
    behind an event, without waiting; the next routed_experts call raises IndexError for every earlier call whose copy
    has landed with the bit set, and check_routing_errors() waits for all of them. No call synchronises the host.
    Under HIP-graph capture nothing is recorded (the replays drop such slots as above)."""

    def __init__(self):
        self.pending = []   # (event, pinned host word)

    def record(self, err: torch.Tensor):
        if torch.cuda.is_current_stream_capturing():
            return
        host = torch.empty(1, dtype=torch.int32, pin_memory=True)
        host.copy_(err, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self.pending.append((ev, host))

    def poll(self, wait: bool = False):
        done, keep = [], []
        for ev, host in self.pending:
            if wait:
                ev.synchronize()
            if wait or ev.query():
                done.append(host)
            else:
                keep.append((ev, host))
        self.pending = keep
        if any(int(h[0]) & 1 for h in done):
            raise IndexError("routed_experts: expert ids must lie in [0, E) (an earlier call's dispatch dropped "
                             "slots with ids out of range)")


_ID_CHECK = _DeferredIdCheck()


def check_routing_errors():
    """Wait for the id checks of earlier routed_experts calls and raise IndexError if any was given an expert id
    outside [0, E) (such slots were dropped: they contributed zero rows)."""
    _ID_CHECK.poll(wait=True)


def routed_experts(x2d, topv, topi, ex: LayerExperts, lora=None):
    """Weighted sum of the routed experts of every token (smel/moe.py:214-252). Expert ids outside [0, E) are reported
    by the next call or check_routing_errors(), without a host synchronisation here."""
    L.require_device(x2d, topv, topi)
    if not torch.cuda.is_current_stream_capturing():
        _ID_CHECK.poll()
    if x2d.dtype == torch.float32:
        return F32.RoutedFn.apply(F32.f32(x2d), topv, topi, ex, lora, _ID_CHECK.record, *_lora_leaves(lora))
    _check_bank(ex)
    if _bf16_limit(x2d.shape[-1], ex, (lora,)) is not None:
        ex32 = _f32_experts(ex, ex.__dict__.setdefault("_dense_packs", {}))
        out = F32.RoutedFn.apply(_bf16(x2d).float(), topv, topi, ex32, lora, _ID_CHECK.record, *_lora_leaves(lora))
        return out.to(x2d.dtype)
    return _RoutedFn.apply(_bf16(x2d), topv, topi, ex, lora, *_lora_leaves(lora))


class _DenseSaved:
    """What the backward of a dense gated MLP needs from its forward."""
    __slots__ = ("x", "actb", "hsave", "ext_gu", "ext_dn", "lb")


def _dense_mlp_fwd(x, w_gu: PackedW, w_dn: PackedW, lb, act_name: str, tag: str = "gemm_mlp"):
    """Gated MLP y = down(act(gate(x)) * up(x)) (+ LoRA on all three as the K-extension) as one dense group of the
    grouped GEMMs (rows = tokens). Returns (y [T, H] bf16, _DenseSaved)."""
    T, H = x.shape
    Is = w_dn.C
    dev = x.device
    st = L.stream()
    tiles, ntiles, maxt, gk = _dense_tiles(T, dev)
    tl = (tiles, ntiles, maxt, gk)
    bf = lambda *s: torch.empty(*s, dtype=torch.bfloat16, device=dev)
    g = lambda n: getattr(lb, n) if lb is not None else None
    planes = lb.planes if lb is not None else 1
    sv = _DenseSaved()
    sv.x, sv.lb, sv.ext_gu, sv.ext_dn = x, lb, None, None
    if lb is not None:
        sv.ext_gu = _lora_ext(tl, x, H, T, 0, None, 0, 1, None, lb, "a_gu", H, planes, T, dev, st)
    sv.actb, sv.hsave = bf(T, Is), bf(T, 2 * Is)
    wg = _dense_wset(w_gu, g("fwd_gu"), planes)
    L.call("smel_gmm_fwd", ctypes.byref(wg), L.ptr(gk), L.ptr(tiles), L.ptr(ntiles), maxt, L.ptr(x), H, T, 0,
           None, 0, 1, L.ptr(sv.ext_gu), 1, _ACT[act_name], L.ptr(sv.actb), Is, L.ptr(sv.hsave), st,
           tag=tag + "_gu_fwd")
    if lb is not None:
        sv.ext_dn = _lora_ext(tl, sv.actb, Is, T, 0, None, 0, 1, None, lb, "a_dn", Is, 1, T, dev, st)
    y = bf(T, H)
    wd = _dense_wset(w_dn, g("fwd_dn"))
    L.call("smel_gmm_fwd", ctypes.byref(wd), L.ptr(gk), L.ptr(tiles), L.ptr(ntiles), maxt, L.ptr(sv.actb), Is, T, 0,
           None, 0, 1, L.ptr(sv.ext_dn), 0, _ACT[act_name], L.ptr(y), H, None, st, tag=tag + "_dn_fwd")
    return y, sv


def _dense_mlp_bwd(sv: _DenseSaved, dy, w_gu_t: PackedW, w_dn_t: PackedW, lora, act_name: str, row_w,
                   tag: str = "gemm_mlp"):
    """Backward of _dense_mlp_fwd for the output row_w[t] * y[t] (row_w fp32 [T]: ones for a plain MLP, the shared
    gate for the shared expert): returns (dx [T, H] bf16, {LoRA name: grad} or None, dwp [T][nblk] fp32 = the
    per-column-block partials of <y[t], dy[t]>, i.e. d loss / d row_w[t], nblk)."""
    x, lb = sv.x, sv.lb
    dy = _bf16(dy)
    T, H = x.shape
    Is = w_dn_t.C
    dev = x.device
    st = L.stream()
    tiles, ntiles, maxt, gk = _dense_tiles(T, dev)
    tl = (tiles, ntiles, maxt, gk)
    bf = lambda *s: torch.empty(*s, dtype=torch.bfloat16, device=dev)
    g = lambda n: getattr(lb, n) if lb is not None else None
    planes = lb.planes if lb is not None else 1
    ext_db = ext_dxa = None
    if lb is not None:
        ext_db = _lora_ext(tl, dy, H, T, 0, None, 0, 1, None, lb, "bt_dn", H, 1, T, dev, st)
    nblk = L.load().smel_gmm_bwd_nblocks(Is)
    dh = bf(T, 2 * Is)
    dwp = torch.empty(T, nblk, dtype=torch.float32, device=dev)
    wd = _dense_wset(w_dn_t, g("at_dn"))
    lrows = _bwd_lora_rows(None, lb, nblk, T, planes, dev) if lb is not None and _BWD_LORA_ROWS else None
    lr = ctypes.byref(lrows[0]) if lrows is not None else None
    L.call("smel_gmm_bwd_lr", ctypes.byref(wd), L.ptr(gk), L.ptr(tiles), L.ptr(ntiles), maxt, L.ptr(dy), H, T, 0,
           None, 0, 1, L.ptr(ext_db), 1, _ACT[act_name], L.ptr(sv.hsave), None, L.ptr(row_w), L.ptr(dh), 2 * Is,
           L.ptr(dwp), lr, st, tag=tag + "_dn_bwd")
    if lb is not None and lrows is None:
        ext_dxa = _lora_ext(tl, dh, 2 * Is, T, 0, None, 0, 1, None, lb, "bt_gu", 2 * Is, planes, T, dev, st)
    dx = bf(T, H)
    wg = _dense_wset(w_gu_t, g("at_gu"), planes)
    L.call("smel_gmm_bwd_lr", ctypes.byref(wg), L.ptr(gk), L.ptr(tiles), L.ptr(ntiles), maxt, L.ptr(dh), 2 * Is, T,
           0, None, 0, 1, None if lrows is not None else L.ptr(ext_dxa), 0, 0, None, None, None, L.ptr(dx), H, None,
           lr, st, tag=tag + "_gu_bwd")
    grads = None
    if lb is not None:
        if lrows is not None:   # the LoRA gradients take the same rows the gate_up backward summed
            ext_dxa = _lora_rows_sum(tl, lrows[0], None, lb, T, planes, dev, st)
        zero = torch.zeros(2, dtype=torch.int32, device=dev)     # offsets of zero experts
        groups = torch.zeros(1, dtype=torch.int32, device=dev)   # group 0 >= E = 0: rows [0, T)
        gs = _alloc_lora_grads(lora, dev)
        # the down projection's products take the row weight (dh already carries it)
        jobs, nj = _wgrad_jobs(H, Is, (None, gs), (None, lora), (ext_dxa, x, T, 0, 0), (sv.ext_gu, dh, T, 0, 0),
                               (ext_db, sv.actb, T, 0, 1), (sv.ext_dn, dy, T, 0, 1), planes)
        ws = _wgrad_ws(jobs, nj, 1, T, dev)
        L.call("smel_lora_wgrad", jobs, nj, L.ptr(groups), 1, 0, L.ptr(zero), 0, T, 0, 1, None, None, L.ptr(row_w),
               T, L.ptr(ws), ws.numel(), st, tag="lora_wgrad")
        grads = gs
    return dx, grads, dwp, nblk


class _MLPFn(torch.autograd.Function):
    """Gated MLP with LoRA on gate/up/down (mlp_lora, smel/moe.py:183-194) as one dense group of the grouped GEMMs:
    rows = tokens, weights = the stacked gate_up [2Is, H] and down [H, Is], each given as (forward layout, transposed
    layout) packs."""

    @staticmethod
    def forward(ctx, x, w_gu2, w_dn2, lora, act_name, *leaves):
        lb = _LoRABufs(lora, 1, x.shape[1], w_dn2[0].C, x.device, _lora_planes(lora)) if lora is not None else None
        y, sv = _dense_mlp_fwd(x, w_gu2[0], w_dn2[0], lb, act_name)
        ctx.sv, ctx.w, ctx.lora, ctx.act_name = sv, (w_gu2[1], w_dn2[1]), lora, act_name
        return y

    @staticmethod
    def backward(ctx, dy):
        sv, (w_gu_t, w_dn_t), lora = ctx.sv, ctx.w, ctx.lora
        ones = torch.ones(sv.x.shape[0], dtype=torch.float32, device=dy.device)   # row weight 1
        dx, gs, _, _ = _dense_mlp_bwd(sv, dy, w_gu_t, w_dn_t, lora, ctx.act_name, ones)
        grads = [gs.get(n) for n in _LORA_NAMES] if gs is not None else [None] * 6
        ctx.sv = ctx.w = ctx.lora = None
        return (dx, None, None, None, None, *grads)


def _dense_wset(w: PackedW, ext, planes: int = 1) -> L.WSet:
    """smel_wset of a dense MLP projection (the shared group); planes = 2 for a two-plane gate_up LoRA."""
    ws = L.WSet()
    ws.wsh = L.ptr(w.t)
    ws.ext_sh = L.ptr(ext)
    ws.R, ws.C, ws.group = w.R, w.C, 32
    if planes == 2:
        ws.flags |= L.WSET_EXT2
    return ws


def mlp_lora(x, w_gate, w_up, w_down, lora, act_name="silu", w_gate_up=None):
    """Gated MLP down(act(gate(x)) * up(x)) with optional LoRA on all three projections (smel/moe.py:183-194),
    as the dense group of the grouped GEMM kernels. x [T, H] bf16; weights bf16."""
    if act_name not in _ACT:
        raise ValueError(f"unknown activation {act_name}")
    L.require_device(x, w_down)
    xs = x.reshape(-1, x.shape[-1])
    to32 = None
    if x.dtype == torch.float32:
        to32 = lambda t, n: None if t is None else F32.f32(t, n)
    elif _bf16_limit(x.shape[-1], None, (lora,), w_down.shape[1]) is not None:
        to32 = lambda t, n: None if t is None else _f32_of(_bf16(t))
    if to32 is not None:
        y = F32.MLPFn.apply(xs.float(), to32(w_gate if w_gate_up is None else None, "w_gate"),
                            to32(w_up if w_gate_up is None else None, "w_up"), to32(w_down, "w_down"),
                            to32(w_gate_up, "w_gate_up"), lora, act_name, *_lora_leaves(lora))
        return y.reshape(*x.shape[:-1], y.shape[-1]).to(x.dtype)
    if w_gate_up is not None:
        gus = (_bf16(w_gate_up),)
        pgu = (_cached("f", lambda: pack_bf16(gus[0]), *gus), _cached("t", lambda: pack_bf16_t(gus[0]), *gus))
    else:
        if w_gate.shape[0] % 32:
            raise L.SmelError(f"mlp_lora: intermediate size {w_gate.shape[0]} must be a multiple of 32")
        gus = (_bf16(w_gate), _bf16(w_up))
        pgu = (_cached("f", lambda: pack_bf16(*gus), *gus), _cached("t", lambda: pack_bf16_t(torch.cat(gus)), *gus))
    dn = _bf16(w_down)
    pdn = (_cached("f", lambda: pack_bf16(dn), dn), _cached("t", lambda: pack_bf16_t(dn), dn))
    y = _MLPFn.apply(_bf16(xs), pgu, pdn, lora, act_name, *_lora_leaves(lora))
    return y.reshape(*x.shape[:-1], y.shape[-1])


def shared_mlp(x, W, lora):
    """smel/moe.py:197-201: the shared expert times sigmoid(x w_sg^T). moe_forward fuses this into its grouped
    GEMMs; this stand-alone form multiplies the gate with torch ops."""
    pre = "mlp.shared_expert."
    y = mlp_lora(x, W.get(pre + "gate_proj.weight"), W.get(pre + "up_proj.weight"), W[pre + "down_proj.weight"], lora,
                 w_gate_up=W.get(pre + "gate_up_proj.weight"))
    if x.dtype == torch.float32:   # the gate as an fp32 GEMM and a HIP kernel
        return F32.GateAddFn.apply(y, F32.f32(x), F32.f32(W["mlp.shared_expert_gate.weight"], "shared gate"), None)
    return y * torch.sigmoid(F.linear(x, W["mlp.shared_expert_gate.weight"]))


def _shared_weights(W: dict, store: dict | None = None):
    """(gate_up, down) of the shared expert packed, the shared-gate row, the shared intermediate size, and (gate_up,
    down) in the backward's transposed layout; None without a shared expert. Packs are reused while the dict's
    tensors are unchanged (kept in ``store``, the layer's own, when given)."""
    pre = "mlp.shared_expert."
    if pre + "gate_proj.weight" not in W and pre + "gate_up_proj.weight" not in W:
        return None
    gu = W.get(pre + "gate_up_proj.weight")
    dn = _bf16(W[pre + "down_proj.weight"])
    if gu is not None:
        gus = (_bf16(gu),)
        pgu = _cached("f", lambda: pack_bf16(gus[0]), *gus, store=store)
        pgu_t = _cached("t", lambda: pack_bf16_t(gus[0]), *gus, store=store)
    else:
        gus = (_bf16(W[pre + "gate_proj.weight"]), _bf16(W[pre + "up_proj.weight"]))
        pgu = _cached("f", lambda: pack_bf16(*gus), *gus, store=store)
        pgu_t = _cached("t", lambda: pack_bf16_t(torch.cat(gus)), *gus, store=store)
    pdn = _cached("f", lambda: pack_bf16(dn), dn, store=store)
    pdn_t = _cached("t", lambda: pack_bf16_t(dn), dn, store=store)
    return pgu, pdn, _bf16(W["mlp.shared_expert_gate.weight"].reshape(-1)), dn.shape[1], pgu_t, pdn_t


def moe_forward(x2d, W, ex: LayerExperts, top_k: int, lora_layer=None, stats=None):
    """x2d [N, H] (already post-attention-normed) -> [N, H] bf16 (smel/moe.py:255-263): router, stats hook, routed
    experts and the shared expert, fused into one forward/backward pipeline."""
    L.require_device(x2d)
    if x2d.dtype == torch.float32:
        return _moe_forward_f32(x2d, W, ex, top_k, lora_layer, stats)
    _check_bank(ex)
    x = _bf16(x2d)
    sh_dn = W.get("mlp.shared_expert.down_proj.weight")
    loras = (lora_layer.experts, lora_layer.shared) if lora_layer is not None else ()
    if _bf16_limit(x.shape[-1], ex, loras, None if sh_dn is None else sh_dn.shape[1]) is not None:
        store = ex.__dict__.setdefault("_dense_packs", {})
        st = None if stats is None else (lambda p, v, i: stats(p, v.to(x.dtype), i))
        return _moe_forward_f32(x.float(), _f32_W(W, store), _f32_experts(ex, store), top_k, lora_layer,
                                st).to(x.dtype)
    lora_ex = lora_layer.experts if lora_layer is not None else None
    lora_sh = lora_layer.shared if lora_layer is not None else None
    store = ex.__dict__.setdefault("_dense_packs", {})   # the layer's shared-expert / router packs live with it
    shared = _shared_weights(W, store)
    # a shared expert of the experts' intermediate size is fused into the expert GEMMs; another runs on its own
    split = shared is not None and shared[3] != _expert_I(ex)
    if lora_ex is not None and (ex.sel_ids is None or len(ex._slot) == 0):
        lora_ex = None
    plan = {"ex": ex, "top_k": int(top_k), "gate_w": _bf16(W["mlp.gate.weight"]), "shared": shared, "store": store,
            "split_shared": split, "lora_ex": lora_ex, "lora_sh": lora_sh if shared is not None else None}
    leaves = _lora_leaves(plan["lora_ex"]) + _lora_leaves(plan["lora_sh"])
    plan["need_grad"] = torch.is_grad_enabled() and (x2d.requires_grad or any(p.requires_grad for p in leaves))
    return _MoELayerFn.apply(x, plan, stats, *leaves)


def _moe_forward_f32(x2d, W, ex: LayerExperts, top_k: int, lora_layer, stats):
    """moe_forward on fp32 activations, composed as the reference composes it (smel/moe.py:255-263): route, the stats
    hook, routed_experts, and the shared expert times its gate added to the routed output (one kernel)."""
    probs, topv, topi = route(x2d, W["mlp.gate.weight"], top_k)
    if stats is not None:
        stats(probs, topv, topi)
    lora_ex = lora_layer.experts if lora_layer is not None else None
    lora_sh = lora_layer.shared if lora_layer is not None else None
    routed = routed_experts(x2d, topv, topi, ex, lora_ex)
    pre = "mlp.shared_expert."
    if pre + "down_proj.weight" not in W:
        return routed
    y = mlp_lora(x2d, W.get(pre + "gate_proj.weight"), W.get(pre + "up_proj.weight"), W[pre + "down_proj.weight"],
                 lora_sh, w_gate_up=W.get(pre + "gate_up_proj.weight"))
    return F32.GateAddFn.apply(y, F32.f32(x2d), F32.f32(W["mlp.shared_expert_gate.weight"], "shared gate"), routed)


def _count_tiles(counts: list, device, order: str = "group"):
    """Tile list of 128-row tiles over contiguous row groups of the given (host) sizes: rows of group e are
    [sum(counts[:e]), +counts[e]). order "group": in group order; "long": the tiles of more than 64 rows first, then
    the short ones (as smel_dispatch's tiles); "merged": a group's last tile of at most 32 rows joined to its full
    tile, then that merged-first, long, short order (as smel_dispatch's tiles_merged, every group of the int4 kind).
    Returns (tiles, n_tiles, max_tiles) as the grouped GEMMs take them."""
    tl, row = [], 0
    merged, long_, short = [], [], []
    for e, c in enumerate(counts):
        t = [(e, r0, min(row + c, r0 + M_TILE), 0) for r0 in range(row, row + c, M_TILE)]
        row += c
        if order == "group":
            tl += t
            continue
        if order == "merged" and len(t) >= 2 and t[-1][2] - t[-1][1] <= M_MERGED - M_TILE:
            last, full = t.pop(), t.pop()
            merged.append((e, full[1], last[2], 0))
        for x in t:
            (long_ if x[2] - x[1] > M_TILE // 2 else short).append(x)
    if order != "group":
        tl = merged + long_ + short
    n = len(tl)
    t = torch.tensor(tl or [(0, 0, 0, 0)], dtype=torch.int32).reshape(-1).to(device)
    return t, torch.tensor([n], dtype=torch.int32).to(device), n


def _bank_gkind(bank, device) -> torch.Tensor:
    """Group kinds of a bare frozen bank: group e = expert e of the bank."""
    cache = bank.__dict__.setdefault("_gkind_plain", {})
    if str(device) not in cache:
        kind = L.KIND_INT4 if isinstance(bank, Int4Experts) else L.KIND_BF16
        cache[str(device)] = torch.tensor([(kind << 16) | e for e in range(bank.num_experts)], dtype=torch.int32,
                                          device=device)
    return cache[str(device)]


class FrozenExpertsFn(torch.autograd.Function):
    """Frozen experts over rows already sorted by expert (smel/moe.py:110-143): ``apply(xs, counts, bank, group,
    act_name)`` with ``counts`` the host list of rows per expert. Forward = the grouped gate_up GEMM (int4 dequant in
    registers or bf16 bank, act-gate epilogue) and the grouped down GEMM; backward = the down-backward GEMM fused with
    the act-gate backward and the gate_up-backward GEMM (weights re-dequantized, no weight gradients). ``group`` (the
    reference's experts-dequantized-at-once knob) is accepted and not needed. The gate/up pre-activations are kept
    from the forward (bf16, the values the reference recomputes) instead of being recomputed."""

    @staticmethod
    def forward(ctx, xs, counts, bank, group, act_name="silu"):
        if act_name not in _ACT:
            raise ValueError(f"unknown activation {act_name}")
        L.require_device(xs)
        ctx.plan = ctx.plan_f32 = None
        ctx.dtype = xs.dtype
        if xs.dtype == torch.float32 or _bf16_limit(xs.shape[-1], bank) is not None:
            counts = [int(c) for c in counts]
            if len(counts) != bank.num_experts or sum(counts) != xs.shape[0] or min(counts, default=0) < 0:
                raise ValueError(f"FrozenExpertsFn: counts (sum {sum(counts)}, {len(counts)} experts) do not match "
                                 f"xs rows {xs.shape[0]} / bank experts {bank.num_experts}")
            if xs.dtype == torch.float32:
                out, ctx.plan_f32 = F32.frozen_fwd(F32.f32(xs), counts, bank, act_name)
                return out
            bank32 = _f32_bank(bank, bank.__dict__.setdefault("_f32_store", {}))
            out, ctx.plan_f32 = F32.frozen_fwd(_bf16(xs).float(), counts, bank32, act_name)
            return out.to(xs.dtype)
        _check_bank(bank)
        xs = _bf16(xs)
        counts = [int(c) for c in counts]
        rows, H = xs.shape
        if len(counts) != bank.num_experts or sum(counts) != rows or min(counts, default=0) < 0:
            raise ValueError(f"FrozenExpertsFn: counts (sum {sum(counts)}, {len(counts)} experts) do not match "
                             f"xs rows {rows} / bank experts {bank.num_experts}")
        dev = xs.device
        st = L.stream()
        w_gu, w_dn = _bank_wset(bank, "gu"), _bank_wset(bank, "dn")
        # the forward GEMMs on the merged list (int4 banks in the fast form, K a multiple of 64), the backward on the
        # long-first list, as in the fused layer
        I = w_dn.C
        merge = _MERGE_SHORT and isinstance(bank, Int4Experts) and (w_gu.flags & L.WSET_FAST_DQ) and H % 64 == 0
        merge_dn = merge and (w_dn.flags & L.WSET_FAST_DQ) and I % 64 == 0
        if merge:
            w_gu.flags |= L.WSET_MERGED_LIST
        if merge_dn:
            w_dn.flags |= L.WSET_MERGED_LIST
        bf = lambda *s: torch.empty(*s, dtype=torch.bfloat16, device=dev)
        out = bf(rows, H)
        ctx.plan = None
        if rows == 0:
            return out
        tiles, ntiles, maxt = _count_tiles(counts, dev, "long")
        tiles_gu, ntiles_gu, maxt_gu = _count_tiles(counts, dev, "merged") if merge else (tiles, ntiles, maxt)
        gk = _bank_gkind(bank, dev)
        actb, hsave = bf(rows, I), bf(rows, 2 * I)
        L.call("smel_gmm_fwd", ctypes.byref(w_gu), L.ptr(gk), L.ptr(tiles_gu), L.ptr(ntiles_gu), maxt_gu, L.ptr(xs), H,
               rows, 0, None, 0, 1, None, 1, _ACT[act_name], L.ptr(actb), I, L.ptr(hsave), st, tag="gemm_frozen_gu_fwd")
        tl_dn = (tiles_gu, ntiles_gu, maxt_gu) if merge_dn else (tiles, ntiles, maxt)
        L.call("smel_gmm_fwd", ctypes.byref(w_dn), L.ptr(gk), L.ptr(tl_dn[0]), L.ptr(tl_dn[1]), tl_dn[2], L.ptr(actb),
               I, rows, 0, None, 0, 1, None, 0, _ACT[act_name], L.ptr(out), H, None, st, tag="gemm_frozen_dn_fwd")
        ctx.plan = (bank, tiles, ntiles, maxt, gk, hsave, act_name)
        return out

    @staticmethod
    def backward(ctx, dy):
        if ctx.plan_f32 is not None:
            keep, ctx.plan_f32 = ctx.plan_f32, None
            return F32.frozen_bwd(keep, dy.float()).to(ctx.dtype), None, None, None, None
        if ctx.plan is None:
            return torch.zeros_like(dy), None, None, None, None
        bank, tiles, ntiles, maxt, gk, hsave, act_name = ctx.plan
        ctx.plan = None
        dy = _bf16(dy)
        rows, H = dy.shape
        dev = dy.device
        st = L.stream()
        w_gu, w_dn = _bank_wset(bank, "gu", t=True), _bank_wset(bank, "dn", t=True)
        I = w_dn.C
        nblk = L.load().smel_gmm_bwd_nblocks(I)
        dh = torch.empty(rows, 2 * I, dtype=torch.bfloat16, device=dev)
        dwp = torch.empty(rows, nblk, dtype=torch.float32, device=dev)
        ones = torch.ones(rows, dtype=torch.float32, device=dev)    # row weight 1 (no combine weight here)
        L.call("smel_gmm_bwd", ctypes.byref(w_dn), L.ptr(gk), L.ptr(tiles), L.ptr(ntiles), maxt, L.ptr(dy), H, rows, 0,
               None, 0, 1, None, 1, _ACT[act_name], L.ptr(hsave), None, L.ptr(ones), L.ptr(dh), 2 * I, L.ptr(dwp),
               st, tag="gemm_frozen_dn_bwd")
        dx = torch.empty(rows, H, dtype=torch.bfloat16, device=dev)
        L.call("smel_gmm_bwd", ctypes.byref(w_gu), L.ptr(gk), L.ptr(tiles), L.ptr(ntiles), maxt, L.ptr(dh), 2 * I,
               rows, 0, None, 0, 1, None, 0, _ACT[act_name], None, None, None, L.ptr(dx), H, None, st,
               tag="gemm_frozen_gu_bwd")
        return dx, None, None, None, None


def frozen_experts_forward(xs, counts, bank, group, act_name="silu"):
    """smel/moe.py:110-117 (no autograd)."""
    with torch.no_grad():
        return FrozenExpertsFn.apply(xs, counts, bank, group, act_name)
