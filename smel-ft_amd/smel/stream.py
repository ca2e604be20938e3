"""Layer weight sources with prefetch for the layer-major runner (the reference's smel/stream.py:1-214), built on
the stager of include/smel_stream.h.

A layer's tensors live in one pinned host arena (``PinnedLayer``: the reference's tensor names, 256-byte aligned
offsets, the dense gate and up projections next to each other). ``prefetch(l)`` copies the arena into a device slot
on copy streams (chunked over two DMA queues) in copy groups: the int4 banks in chunks of BANK_CHUNK experts first,
then the selected experts, then the rest. A pack stream turns each group into the grouped GEMMs' layouts as soon as
its copies have landed (forward and transposed int4 layouts, the selected experts' bf16 layouts), writing into a
second arena the slot owns, so an upload allocates nothing on the device and only the last group's packing follows
the copy; ``get(l)`` makes the current (compute) stream wait on the stage's event. The host never blocks on a copy
(the reference's worker thread waits on every upload's event, smel/stream.py:62). The one host synchronisation is the
exact-fast-dequant check of an int4 bank, once per pinned layer before its first upload (the answer is kept with the
pinned layer).

Differences from the reference, by design: a slot is reused once ``max_on_gpu`` other layers were fetched after it,
so a ``LayerWeights`` from ``get(l)`` is valid until then (the layer-major runner uses a layer before fetching the
next ones); device memory is a fixed set of slots (no allocator churn per layer).
"""
from __future__ import annotations

import ctypes
import itertools
import json
import os
import time
from collections import OrderedDict

import torch
from safetensors.torch import load_file as load_safetensors

from . import _lib as L
from .moe import BF16Experts, Int4Experts, LayerExperts, PackedW

ALIGN = 256
CHUNK_BYTES = 8 << 20
N_COPY_STREAMS = 2
BANK_CHUNK = 64          # experts per copy group of an int4 bank (each group is packed as soon as it has landed)


class LayerWeights:
    """Device tensors of one decoder layer: dense part (names relative to the layer) + routed experts
    (smel/layer_runner.py:265-278). Gate and up of the dense / shared MLP are presented stacked as
    ``*gate_up_proj.weight`` with the old names as views; when they are adjacent in memory (as a ``PinnedLayer``
    stages them) the stacked tensor is a view too, otherwise one concatenation."""

    def __init__(self, idx: int, ltype: str, W: dict, experts: LayerExperts):
        W = dict(W)
        for pre in ("mlp.shared_expert.", "mlp."):
            g, u = W.get(pre + "gate_proj.weight"), W.get(pre + "up_proj.weight")
            if g is not None and u is not None and g.shape == u.shape and g.dtype == u.dtype:
                if (g.is_contiguous() and u.is_contiguous() and g.untyped_storage().data_ptr()
                        == u.untyped_storage().data_ptr() and u.data_ptr() == g.data_ptr() + g.numel() * g.element_size()):
                    gu = torch.as_strided(g, (2 * g.shape[0],) + tuple(g.shape[1:]), g.stride())
                else:
                    gu = torch.cat((g, u))
                W[pre + "gate_up_proj.weight"], W[pre + "gate_proj.weight"], W[pre + "up_proj.weight"] = \
                    gu, gu[:g.shape[0]], gu[g.shape[0]:]
        self.idx, self.ltype, self.W, self.experts = idx, ltype, W, experts


_EXPERT_PREFIXES = ("mlp.experts.", "experts.")   # routed-expert tensors; everything else is the dense part
_SEL_PREFIX = "experts.sel."


def _id_list(ids) -> list:
    """Expert ids (list, tuple, tensor or None) as a list of Python ints."""
    if ids is None:
        return []
    if isinstance(ids, torch.Tensor):
        ids = ids.reshape(-1).tolist()
    return [int(i) for i in ids]


def _fused_bank(bank: dict, sel_ids):
    """bf16 fused bank [E, 2I, H] / [E, H, I]: the frozen experts, and trainable copies of the selected rows."""
    gu, dn = bank["mlp.experts.gate_up_proj"], bank["mlp.experts.down_proj"]
    ids = _id_list(sel_ids)
    if not ids:
        return BF16Experts(gu, dn), None, None, None
    pick = torch.tensor(ids, dtype=torch.long, device=gu.device)
    return BF16Experts(gu, dn), sel_ids, gu.index_select(0, pick), dn.index_select(0, pick)


def _packed_bank(bank: dict, sel_ids, frozen_dtype):
    """Packed int4 bank ('experts.{gate_up,down}.{q,scale,zero}') with the packed block's own bf16 selection
    ('experts.sel.*'); ``sel_ids`` overrides the block's id list."""
    halves = {w: {} for w in ("gate_up", "down")}
    for k, v in bank.items():
        which, _, field = k[len("experts."):].partition(".")
        if which in halves:
            halves[which][field] = v
    sel_gu, sel_dn = bank.get(_SEL_PREFIX + "gate_up"), bank.get(_SEL_PREFIX + "down")
    if sel_gu is None:
        return Int4Experts(halves["gate_up"], halves["down"], dtype=frozen_dtype), None, None, None
    if sel_ids is None:
        sel_ids = _id_list(bank.get(_SEL_PREFIX + "ids")) or None
    return Int4Experts(halves["gate_up"], halves["down"], dtype=frozen_dtype), sel_ids, sel_gu, sel_dn


def build_layer(idx, ltype, t: dict, sel_ids=None, group=32, frozen_dtype=torch.bfloat16, act="silu"):
    """LayerWeights of one layer from its device tensors (names relative to the layer), smel/stream.py:16-36: the
    routed experts come either as the bf16 fused bank ('mlp.experts.gate_up_proj' / 'down_proj', the selected
    experts copied out of it) or as the packed int4 bank with its selection ('experts.*'); the rest is the dense
    part. Without selected bf16 experts the layer has no selection."""
    dense, bank = {}, {}
    for k, v in t.items():
        (bank if k.startswith(_EXPERT_PREFIXES) else dense)[k] = v
    if "mlp.experts.gate_up_proj" in bank:
        frozen, ids, sel_gu, sel_dn = _fused_bank(bank, sel_ids)
    else:
        frozen, ids, sel_gu, sel_dn = _packed_bank(bank, sel_ids, frozen_dtype)
    return LayerWeights(idx, ltype, dense, LayerExperts(frozen, ids, sel_gu, sel_dn, group=group, act=act))


def _order(names):
    """Staging order: every name in sorted order, except that an MLP's up projection follows its gate projection."""
    out = []
    for k in sorted(names):
        if k.endswith("up_proj.weight") and k.replace("up_proj", "gate_proj") in names:
            continue
        out.append(k)
        if k.endswith("gate_proj.weight") and k.replace("gate_proj", "up_proj") in names:
            out.append(k.replace("gate_proj", "up_proj"))
    return out


def arena_layout(t: dict):
    """{name: (offset, shape, dtype, nbytes)} and the total size of a layer's arena (offsets aligned to ALIGN except
    an up projection, which directly follows its gate projection when that keeps its alignment)."""
    meta, off = OrderedDict(), 0
    for k in _order(list(t)):
        v = t[k]
        nb = v.numel() * v.element_size()
        glued = k.endswith("up_proj.weight") and k.replace("up_proj", "gate_proj") in meta
        if not glued or off % v.element_size():
            off = -(-off // ALIGN) * ALIGN
        meta[k] = (off, tuple(v.shape), v.dtype, nb)
        off += nb
    return meta, -(-off // ALIGN) * ALIGN


def bank_geometry(meta: dict) -> dict:
    """{'gu' | 'dn': (E, R, C, group)} of the int4 banks an arena layout holds (q [E][R][C/2], scale / zero
    [E][R][C/group])."""
    banks = {}
    for which, name in (("gu", "gate_up"), ("dn", "down")):
        q, sc = meta.get(f"experts.{name}.q"), meta.get(f"experts.{name}.scale")
        if q is not None and sc is not None and f"experts.{name}.zero" in meta:
            E, R, half = q[1]
            banks[which] = (E, R, 2 * half, 2 * half // sc[1][2])
    return banks


class PinnedLayer:
    """One layer's tensors copied once into a pinned host arena (page-locked: the DMA engines read it directly)."""

    def __init__(self, t: dict):
        self.meta, self.nbytes = arena_layout(t)
        self.host = torch.empty(max(self.nbytes, ALIGN), dtype=torch.uint8, pin_memory=True)
        for k, (off, _, _, nb) in self.meta.items():
            if nb:
                self.host[off:off + nb].copy_(t[k].detach().contiguous().reshape(-1).view(torch.uint8))
        ids = t.get("experts.sel.ids")
        self.sel_ids = None if ids is None else [int(i) for i in ids.tolist()]
        self.fast = {}   # int4 bank: {'gu' | 'dn': exact fast dequant form holds}, filled before the first upload
        self.banks = bank_geometry(self.meta)


_BANK_NAMES = {"gu": "gate_up", "dn": "down"}


class _UploadPlan:
    """How a pinned layer goes up: its copy groups (lists of (arena offset, bytes)) in order, what is packed after
    each, and the byte layout of the packed GEMM layouts in the slot's pack arena."""

    def __init__(self, P: PinnedLayer):
        lib = L.load()
        self.groups, self.after = [], []          # after[i]: ('bank', which, e0, e1) / ('sel',) / None
        self.pack_at, self.pack_bytes = {}, 0     # name -> (byte offset, bytes) in the pack arena

        def put(name, nb):
            self.pack_at[name] = (self.pack_bytes, nb)
            self.pack_bytes += -(-nb // ALIGN) * ALIGN

        banked = set()
        for which, (E, R, C, g) in P.banks.items():
            fields = [P.meta[f"experts.{_BANK_NAMES[which]}.{f}"] for f in ("q", "scale", "zero")]
            banked.update(f"experts.{_BANK_NAMES[which]}.{f}" for f in ("q", "scale", "zero"))
            for e0 in range(0, E, BANK_CHUNK):
                e1 = min(E, e0 + BANK_CHUNK)
                self.groups.append([(off + e0 * (nb // E), (e1 - e0) * (nb // E)) for off, _, _, nb in fields])
                self.after.append(("bank", which, e0, e1))
            put(which + ".f.q", lib.smel_packed_bytes(L.PACK_Q4, E * R, C))
            put(which + ".f.sz", lib.smel_packed_bytes(L.PACK_SZ, E * R, C))
            put(which + ".t.q", lib.smel_packed_t_bytes(L.PACK_Q4, E, R, C, g))
            put(which + ".t.sz", lib.smel_packed_t_bytes(L.PACK_SZ, E, R, C, g))
        sel = [k for k in ("experts.sel.gate_up", "experts.sel.down") if k in P.meta]
        if P.banks and len(sel) == 2 and P.sel_ids:
            self.groups.append([P.meta[k][0:1] + (P.meta[k][3],) for k in sel])
            self.after.append(("sel",))
            banked.update(sel)
            for k in sel:
                n, R, C = P.meta[k][1]
                put(k + ".f", lib.smel_packed_bytes(L.PACK_BF16, n * R, C))
                put(k + ".t", lib.smel_packed_t_bytes(L.PACK_BF16, n, R, C, 0))
        rest = sorted((off, nb) for k, (off, _, _, nb) in P.meta.items() if k not in banked and nb)
        runs = []
        for off, nb in rest:   # neighbours (up to alignment padding) go as one region
            if runs and off - (runs[-1][0] + runs[-1][1]) < ALIGN:
                runs[-1] = (runs[-1][0], off + nb - runs[-1][0])
            else:
                runs.append((off, nb))
        if runs:
            self.groups.append(runs)
            self.after.append(None)


class _Slot:
    def __init__(self, nbytes, device):
        self.device = device
        self.arena = torch.empty(max(nbytes, ALIGN), dtype=torch.uint8, device=device)
        self.pack = torch.empty(ALIGN, dtype=torch.uint8, device=device)   # the staged layer's packed layouts
        self.free = _Event()                 # recorded on the compute stream when the slot is given up
        self.free_used = False
        self.done = []                       # [copy group][copy stream] events, made as needed
        self.ready = _Event()
        self.layer = None
        self.LW = None

    def group_events(self, n: int):
        while len(self.done) < n:
            self.done.append([_Event() for _ in range(N_COPY_STREAMS)])
        return self.done[:n]

    def pack_arena(self, nbytes: int) -> torch.Tensor:
        """The pack arena, grown if a layer needs more (freed blocks are reused in the compute stream's order)."""
        if self.pack.numel() < nbytes:
            self.pack = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        return self.pack


class _Event:
    """A timing-free HIP event owned by the library (smel_event_create)."""

    def __init__(self):
        h = ctypes.c_void_p()
        L.call("smel_event_create", ctypes.byref(h))
        self.h = h

    def __del__(self):
        try:
            if self.h:
                L.load().smel_event_destroy(self.h)
        except Exception:   # interpreter shutdown
            pass


class _StagedSource:
    """prefetch(l) / get(l) -> LayerWeights / close() / stats, as the reference's _StreamingSource
    (smel/stream.py:39-114), over the device slots of the stager. Subclasses give _pinned(l) -> PinnedLayer and
    _ltype(l)."""

    def __init__(self, device="cuda", resident=False, max_on_gpu=2, group=32, act="silu"):
        self.device = torch.device(device)
        L.require_device(torch.empty(0, device=self.device))
        self.resident, self.max_on_gpu, self.group, self.act = resident, max(1, max_on_gpu), group, act
        self.slots = []                     # _Slot, in least-recently-used order at the front
        self.copy = [torch.cuda.Stream(self.device) for _ in range(N_COPY_STREAMS)]   # default priority
        self.packer = torch.cuda.Stream(self.device)   # packs each copy group as soon as it has landed
        self.stats = {"load_s": 0.0, "wait_s": 0.0, "bytes": 0, "loads": 0}
        self.cache = {}                     # l -> LayerWeights staged (views into a slot)
        # (PinnedLayer, event after its stage): a host arena made for one upload stays referenced until its copies
        # are done, since the DMA reads it behind torch's back and torch would otherwise recycle the pinned block
        self._in_flight = []

    # -- subclass hooks
    def _pinned(self, l) -> PinnedLayer:
        raise NotImplementedError

    def _ltype(self, l) -> str:
        return "linear_attention"

    def _sel_ids(self, l, P: PinnedLayer):
        """The selected experts of layer l: those the layer's own tensors name (``experts.sel.ids``)."""
        return P.sel_ids

    # --
    def _slot_for(self, l, nbytes):
        for s in self.slots:
            if s.layer == l:
                return s, True
        if self.resident or len(self.slots) < self.max_on_gpu:
            s = _Slot(nbytes, self.device)
            self.slots.append(s)
            return s, False
        s = self.slots[0]                   # least recently used
        if s.arena.numel() < nbytes:
            s.arena = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        # every kernel that reads the evicted layer was enqueued on the current stream before this point
        L.call("smel_event_record", s.free.h, L.stream())
        s.free_used = True
        self.cache.pop(s.layer, None)
        s.layer, s.LW = None, None
        return s, False

    def _fast_flags(self, P: PinnedLayer) -> dict:
        """Whether each int4 bank of P admits the GEMMs' exact fast dequant form (smel_int4_fast_ok on its scale /
        zero, uploaded for the check): decided once per pinned layer, before its first upload, with one host
        synchronisation, so that the transposed layouts can be packed chunk by chunk as the copies land."""
        if P.fast or not P.banks:
            return P.fast
        oks = {}
        for which, (E, R, C, g) in P.banks.items():
            name = _BANK_NAMES[which]
            (so, _, _, nb), (zo, _, _, _) = P.meta[f"experts.{name}.scale"], P.meta[f"experts.{name}.zero"]
            sz = torch.empty(2 * nb, dtype=torch.uint8, device=self.device)
            sz[:nb].copy_(P.host[so:so + nb], non_blocking=True)
            sz[nb:].copy_(P.host[zo:zo + nb], non_blocking=True)
            oks[which] = torch.zeros(1, dtype=torch.int32, device=self.device)
            L.call("smel_int4_fast_ok", L.ptr(sz), sz.data_ptr() + nb, nb // 2, L.ptr(oks[which]), L.stream())
        P.fast = {k: bool(v.item()) for k, v in oks.items()}
        return P.fast

    def prefetch(self, l):
        """Stage layer l in a device slot (copies on the copy streams, packing on the pack stream; returns at
        once)."""
        if l in self.cache:
            return
        t0 = time.perf_counter()
        P = self._pinned(l)
        s, hit = self._slot_for(l, P.nbytes)
        if hit:
            return
        fast = self._fast_flags(P)
        plan = _UploadPlan(P)
        pack = s.pack_arena(plan.pack_bytes)
        streams = (ctypes.c_void_p * N_COPY_STREAMS)(*[c.cuda_stream for c in self.copy])
        events = s.group_events(len(plan.groups))
        after = s.free.h if s.free_used else None   # queued kernels may still read the slot's previous layer
        for regions, evs in zip(plan.groups, events):
            arr = (L.H2DRegion * len(regions))(*[L.H2DRegion(s.arena.data_ptr() + off, P.host.data_ptr() + off, nb)
                                                 for off, nb in regions])
            done = (ctypes.c_void_p * N_COPY_STREAMS)(*[e.h for e in evs])
            L.call("smel_h2d_regions", arr, len(regions), CHUNK_BYTES, streams, done, N_COPY_STREAMS, after)
            after = None
        torch.autograd.graph.increment_version(s.arena)   # packed-layout caches keyed on the old bytes miss
        t = {k: s.arena[off:off + nb].view(dt).view(shape) for k, (off, shape, dt, nb) in P.meta.items()}
        pk = self.packer
        if s.free_used:
            L.call("smel_stream_wait", pk.cuda_stream, s.free.h)   # the pack arena is read by those kernels too
        with torch.cuda.stream(pk):
            LW = build_layer(l, self._ltype(l), t, self._sel_ids(l, P), self.group, act=self.act)
            views = {k: pack[o:o + nb] for k, (o, nb) in plan.pack_at.items()}
            for what, evs in zip(plan.after, events):
                for e in evs:
                    L.call("smel_stream_wait", pk.cuda_stream, e.h)
                if what is not None and what[0] == "bank":
                    self._pack_bank_chunk(P, s, views, fast, *what[1:])
                elif what is not None:
                    self._pack_selected(P, s, views)
            self._attach(LW.experts, P, views, fast, plan)
        L.call("smel_event_record", s.ready.h, pk.cuda_stream)
        staged = torch.cuda.Event()
        staged.record(pk)                   # the pack stream has waited on every copy group of this upload
        self._in_flight = [(p, e) for p, e in self._in_flight if not e.query()] + [(P, staged)]
        s.layer, s.LW = l, LW
        self.cache[l] = LW
        self.slots.remove(s)
        self.slots.append(s)
        self.stats["load_s"] += time.perf_counter() - t0
        self.stats["bytes"] += P.nbytes
        self.stats["loads"] += 1

    @staticmethod
    def _pack_bank_chunk(P: PinnedLayer, s: _Slot, views: dict, fast: dict, which: str, e0: int, e1: int):
        """Experts [e0, e1) of an int4 bank into the forward and transposed layouts (smel_pack_int4 / _int4_t), on
        the current (pack) stream."""
        lib = L.load()
        E, R, C, g = P.banks[which]
        name, n = _BANK_NAMES[which], e1 - e0
        q, sc, z = (P.meta[f"experts.{name}.{f}"] for f in ("q", "scale", "zero"))
        src = [s.arena.data_ptr() + off + e0 * (nb // E) for off, _, _, nb in (q, sc, z)]
        fq = views[which + ".f.q"].data_ptr() + lib.smel_packed_bytes(L.PACK_Q4, e0 * R, C)
        fsz = views[which + ".f.sz"].data_ptr() + lib.smel_packed_bytes(L.PACK_SZ, e0 * R, C)
        L.call("smel_pack_int4", *src, n * R, C, g, fq, fsz, L.stream())
        tq = views[which + ".t.q"].data_ptr() + lib.smel_packed_t_bytes(L.PACK_Q4, e0, R, C, g)
        tsz = views[which + ".t.sz"].data_ptr() + lib.smel_packed_t_bytes(L.PACK_SZ, e0, R, C, g)
        L.call("smel_pack_int4_t", *src, n, R, C, g, int(fast[which]), tq, tsz, L.stream())

    @staticmethod
    def _pack_selected(P: PinnedLayer, s: _Slot, views: dict):
        """The selected experts' bf16 gate_up / down into the forward and transposed layouts (smel_pack_bf16 /
        _bf16_t), on the current (pack) stream."""
        for k in ("experts.sel.gate_up", "experts.sel.down"):
            off, (n, R, C), _, _ = P.meta[k]
            w = s.arena.data_ptr() + off
            L.call("smel_pack_bf16", w, n * R, C, C, views[k + ".f"].data_ptr(), L.stream())
            L.call("smel_pack_bf16_t", w, n, R, C, C, views[k + ".t"].data_ptr(), L.stream())

    @staticmethod
    def _attach(ex: LayerExperts, P: PinnedLayer, views: dict, fast: dict, plan: _UploadPlan):
        """Hand the packed layouts in the pack arena to the layer's expert objects (their caches), as the layouts
        their own packing would have built."""
        fz = ex.frozen
        if isinstance(fz, Int4Experts) and P.banks:
            fz._fast_dq = dict(fast)
            fz._packed = {w: (views[w + ".f.q"], views[w + ".f.sz"].view(torch.int32)) for w in P.banks}
            fz._packed_t = {w: (views[w + ".t.q"], views[w + ".t.sz"].view(torch.float32)) for w in P.banks}
        if ("sel",) in plan.after and ex.sel_ids is not None and ex._slot:
            mk = lambda k, sfx: PackedW(views[k + sfx].view(torch.bfloat16), P.meta[k][1][1], P.meta[k][1][2])
            ex._packed_sel = (mk("experts.sel.gate_up", ".f"), mk("experts.sel.down", ".f"))
            ex._packed_sel_t = (mk("experts.sel.gate_up", ".t"), mk("experts.sel.down", ".t"))
        else:   # a bf16 bank, or selected experts outside the plan: their layouts are packed at first use
            ex.packed_sel()
            ex.packed_sel_t()

    @staticmethod
    def _stage_tensors(LW: LayerWeights):
        """Tensors of a staged layer that were allocated on the pack stream (stacked or selected copies, packs made
        there); they must not be reused by the allocator before the compute stream is done with them. The slot
        arenas are the compute stream's own."""
        ex = LW.experts
        out = [v for v in LW.W.values() if isinstance(v, torch.Tensor)]
        out += [v for v in (ex.sel_gate_up, ex.sel_down) if isinstance(v, torch.Tensor)]
        for name in ("_packed_sel", "_packed_sel_t"):
            for p in ex.__dict__.get(name) or ():
                out.append(p.t)
        return out

    def get(self, l) -> LayerWeights:
        """The staged layer l (staged now if it was not prefetched); the current stream waits for its stage."""
        t0 = time.perf_counter()
        if l not in self.cache:
            self.prefetch(l)
        s = next(x for x in self.slots if x.layer == l)
        cur = L.stream()
        L.call("smel_stream_wait", cur, s.ready.h)
        cs = torch.cuda.current_stream(self.device)
        for x in self._stage_tensors(s.LW):   # made on the pack stream, read on this one
            x.record_stream(cs)
        self.slots.remove(s)
        self.slots.append(s)
        self.stats["wait_s"] += time.perf_counter() - t0
        return s.LW

    def close(self):
        torch.cuda.synchronize(self.device)
        self._in_flight.clear()
        self.cache.clear()
        self.slots.clear()


class DictSource:
    """Already materialized LayerWeights (tests / fully resident block), smel/stream.py:200-214."""

    def __init__(self, layers: dict):
        self.layers = layers
        self.stats = {"load_s": 0.0, "wait_s": 0.0, "bytes": 0, "loads": 0}

    def get(self, l):
        return self.layers[l]

    def prefetch(self, l):
        pass

    def close(self):
        pass


class PinnedSource(_StagedSource):
    """Layers given as dicts of CPU tensors (e.g. ``pack_layer`` outputs), pinned once at construction."""

    def __init__(self, layers: dict, ltypes=None, device="cuda", resident=False, max_on_gpu=2, group=32,
                 act="silu"):
        super().__init__(device, resident, max_on_gpu, group, act)
        self.pinned = {l: PinnedLayer(t) for l, t in layers.items()}
        self.ltypes = ltypes or {}

    def _pinned(self, l):
        return self.pinned[l]

    def _ltype(self, l):
        return self.ltypes.get(l, "linear_attention")


PACKED_FILE = "layer_{:02d}.safetensors"   # one file per layer of a packed block


def _override_selection(own: dict, sel_rows, l, conv=None) -> dict:
    """A layer's entries under a new selection: without one (``sel_rows`` None) its own entries; with one, its own
    'experts.sel.*' entries give way to the selection's for layer l (none if the selection leaves it out). ``conv``
    maps the selection's tensors first (e.g. to their sizes)."""
    if sel_rows is None:
        return own
    new = sel_rows.get(l, {})
    out = {k: v for k, v in own.items() if not k.startswith(_SEL_PREFIX)}
    out.update(new if conv is None else {k: conv(v) for k, v in new.items()})
    return out


def _selected_rows(selection: dict, layers, ckpt) -> dict:
    """{l: the packed layer's experts.sel.* tensors} for a new selection, from the original checkpoint's fused bf16
    expert tensors (only the selected rows are read)."""
    rows = {}
    for l in layers:
        ids = [int(e) for e in selection.get(l, [])]
        if not ids:
            continue
        if ckpt is None:
            raise ValueError("PackedSource: a new selection needs ckpt= to read the selected experts' bf16 rows")
        part = {"experts.sel.ids": torch.tensor(ids, dtype=torch.long)}
        for field, short in (("gate_up", "mlp.experts.gate_up_proj"), ("down", "mlp.experts.down_proj")):
            part[f"experts.sel.{field}"] = ckpt.get_rows(ckpt.full_name(l, short), ids).contiguous()
        rows[l] = part
    return rows


class CheckpointSource(_StagedSource):
    """Layers straight from the original checkpoint (smel/stream.py:117-139): ``ckpt`` gives layer(l) (the layer's
    tensors under layer-relative names, bf16 experts fused) and ``dims`` (layer_types, act). frozen="bf16" streams
    the dense and expert tensors in ``dtype`` (SSM A_log / dt_bias and non-floating tensors as they are);
    frozen="int4" packs each layer with pack_layer (int4 bank from the GPU quantizer, group ``quant_group``) before
    it is pinned. The checkpoint reader itself is the caller's."""

    def __init__(self, ckpt, device="cuda", dtype=torch.bfloat16, selection=None, resident=False, group=32,
                 frozen="bf16", quant_group=64, max_on_gpu=2):
        if frozen not in ("bf16", "int4"):
            raise ValueError(f"frozen must be 'bf16' or 'int4', got {frozen!r}")
        super().__init__(device, resident, max_on_gpu, group, getattr(ckpt.dims, "act", "silu"))
        self.ckpt, self.d, self.dtype = ckpt, ckpt.dims, dtype
        self.selection = selection or {}
        self.frozen, self.quant_group = frozen, quant_group

    def _host_layer(self, l) -> dict:
        from .pack import _dense_part, pack_layer
        t = self.ckpt.layer(l)
        if self.frozen == "int4":
            return pack_layer(t, self.selection.get(l), self.quant_group, self.dtype)
        return {**_dense_part(t, self.dtype), **{k: v.to(self.dtype).contiguous() for k, v in t.items()
                                                 if k.startswith("mlp.experts.")}}

    def _pinned(self, l):
        return PinnedLayer(self._host_layer(l))

    def _sel_ids(self, l, P: PinnedLayer):
        ids = self.selection.get(l)
        return P.sel_ids if P.sel_ids is not None else (list(ids) if ids else None)

    def _ltype(self, l):
        return self.d.layer_types[l]


class PackedSource(_StagedSource):
    """Layers from the packed block, one ``layer_{l:02d}.safetensors`` per layer (smel/stream.py:142-197). With
    pin=True every layer is read once into pinned RAM (up to pin_budget_gb); the rest are read and pinned at each
    upload. ``dims`` needs ``layer_types`` and ``act``."""

    def __init__(self, packed_dir, dims, layers, device="cuda", resident=False, pin=False, group=32,
                 pin_budget_gb=9.0, preloaded=None, selection=None, ckpt=None, max_on_gpu=2):
        """selection {l: [expert ids]} + ckpt: train another expert set on the same packed block. The int4 bank holds
        every expert, so only the new selection's bf16 rows are read, once, from the original checkpoint (``ckpt``
        with full_name(l, short) and get_rows(name, ids), the reference's Checkpoint interface); the packed block's
        own ``experts.sel.*`` are then ignored, and a layer left out of ``selection`` trains no routed expert."""
        super().__init__(device, resident, max_on_gpu, group, getattr(dims, "act", "silu"))
        self.dir, self.d = packed_dir, dims
        self.sel_rows = None if selection is None else _selected_rows(selection, layers, ckpt)
        self.preloaded = preloaded or {}
        self.pinned = {}
        used = 0
        if pin:
            # the longest prefix of `layers` whose tensor bytes fit the budget, decided from the files' headers (and
            # the preloaded dicts) before any tensor is read; only those layers are then read and pinned
            fits = itertools.takewhile(lambda lc: lc[1] / 2**30 <= pin_budget_gb,
                                       zip(layers, itertools.accumulate(map(self._layer_bytes, layers))))
            for l, used in list(fits):
                self.pinned[l] = PinnedLayer(self._layer_tensors(l))
                self.preloaded.pop(l, None)   # the pinned arena replaces the caller's host copy
        self.pinned_gb = used / 2**30

    def _file(self, l) -> str:
        return os.path.join(self.dir, PACKED_FILE.format(l))

    def _own_tensor_bytes(self, l) -> dict:
        """{name: bytes} of layer l's own tensors (preloaded dict, or the safetensors header of its file)."""
        if l in self.preloaded:
            return {k: v.numel() * v.element_size() for k, v in self.preloaded[l].items()}
        with open(self._file(l), "rb") as f:
            n = int.from_bytes(f.read(8), "little")
            head = json.loads(f.read(n))
        return {k: e["data_offsets"][1] - e["data_offsets"][0] for k, e in head.items() if k != "__metadata__"}

    def _layer_bytes(self, l) -> int:
        sizes = _override_selection(self._own_tensor_bytes(l), self.sel_rows, l,
                                    lambda v: v.numel() * v.element_size())
        return sum(sizes.values())

    def _layer_tensors(self, l) -> dict:
        """Host tensors of layer l: the preloaded dict or the whole file, with a new selection's rows in place of the
        packed block's own."""
        own = self.preloaded[l] if l in self.preloaded else load_safetensors(self._file(l))
        return _override_selection(own, self.sel_rows, l)

    def _pinned(self, l):
        P = self.pinned.get(l)
        return P if P is not None else PinnedLayer(self._layer_tensors(l))

    def _ltype(self, l):
        return self.d.layer_types[l]
