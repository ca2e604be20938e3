"""Host side of layer streaming (CPU only): the pinned arena layout (every tensor inside, aligned, no overlap, an
MLP's up projection right after its gate projection) and the argument checks of the stager's C-ABI entry points
(each case fails before any HIP call)."""
import ctypes

import torch

from smel import _lib
from smel.stream import ALIGN, arena_layout


def test_arena_layout():
    t = {"mlp.shared_expert.up_proj.weight": torch.zeros(96, 64, dtype=torch.bfloat16),
         "mlp.shared_expert.gate_proj.weight": torch.zeros(96, 64, dtype=torch.bfloat16),
         "experts.gate_up.q": torch.zeros(4, 10, 7, dtype=torch.uint8),
         "experts.sel.ids": torch.zeros(3, dtype=torch.int64), "odd": torch.zeros(5, dtype=torch.bfloat16),
         "empty": torch.zeros(0, dtype=torch.float32)}
    meta, total = arena_layout(t)
    assert set(meta) == set(t) and total % ALIGN == 0
    spans = sorted((off, off + nb) for off, _, _, nb in meta.values())
    assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:])) and spans[-1][1] <= total
    for k, (off, shape, dt, nb) in meta.items():
        assert shape == tuple(t[k].shape) and dt == t[k].dtype and nb == t[k].numel() * t[k].element_size()
        if k != "mlp.shared_expert.up_proj.weight":
            assert off % ALIGN == 0
    g, u = meta["mlp.shared_expert.gate_proj.weight"], meta["mlp.shared_expert.up_proj.weight"]
    assert u[0] == g[0] + g[3]


def test_stager_entry_points_reject_bad_arguments():
    L = _lib.load()
    EINVAL = -1
    assert L.smel_event_create(None) == EINVAL
    assert L.smel_event_record(None, None) == EINVAL
    assert L.smel_stream_wait(None, None) == EINVAL
    fake = ctypes.c_void_p(1 << 20)   # never dereferenced
    reg = (_lib.H2DRegion * 1)(_lib.H2DRegion(None, fake, 64))
    streams = (ctypes.c_void_p * 2)(None, None)
    done = (ctypes.c_void_p * 2)(fake, fake)
    assert L.smel_h2d_regions(reg, 1, 1 << 20, streams, done, 2, None) == EINVAL       # null destination
    reg_ok = (_lib.H2DRegion * 1)(_lib.H2DRegion(fake, fake, 64))
    assert L.smel_h2d_regions(reg_ok, 1, 0, streams, done, 2, None) == EINVAL          # chunk size 0
    assert L.smel_h2d_regions(reg_ok, 1, 1 << 20, streams, done, 0, None) == EINVAL    # no copy stream
    assert L.smel_h2d_regions(reg_ok, 1, 1 << 20, streams, done, 9, None) == EINVAL    # too many
    nodone = (ctypes.c_void_p * 2)(fake, None)
    assert L.smel_h2d_regions(reg_ok, 1, 1 << 20, streams, nodone, 2, None) == EINVAL  # a null done event
    assert L.smel_h2d_regions(reg_ok, -1, 1 << 20, streams, done, 2, None) == EINVAL


class _FakePinned:
    """The parts of a PinnedLayer the upload plan reads (its constructor needs pinned, i.e. GPU-backed, memory)."""

    def __init__(self, t, sel_ids):
        from smel.stream import bank_geometry
        self.meta, self.nbytes = arena_layout(t)
        self.sel_ids = sel_ids
        self.banks = bank_geometry(self.meta)


def test_upload_plan_covers_the_arena():
    """The copy groups of an upload (int4 banks in chunks of BANK_CHUNK experts, then the selected experts, then the
    rest) cover every byte of every tensor exactly once and nothing else outside alignment padding; the bank groups
    come first, in expert order, each followed by the packing of its experts; the pack arena holds every packed
    layout, each of the size the size queries give."""
    from smel import stream
    E, I, H, g, n = 130, 64, 128, 64, 3   # 130 experts: chunks of 64, 64 and 2
    bf, u8 = torch.bfloat16, torch.uint8
    t = {"experts.gate_up.q": torch.zeros(E, 2 * I, H // 2, dtype=u8),
         "experts.gate_up.scale": torch.zeros(E, 2 * I, H // g, dtype=bf),
         "experts.gate_up.zero": torch.zeros(E, 2 * I, H // g, dtype=bf),
         "experts.down.q": torch.zeros(E, H, I // 2, dtype=u8),
         "experts.down.scale": torch.zeros(E, H, I // g, dtype=bf), "experts.down.zero": torch.zeros(E, H, I // g, dtype=bf),
         "experts.sel.ids": torch.arange(n), "experts.sel.gate_up": torch.zeros(n, 2 * I, H, dtype=bf),
         "experts.sel.down": torch.zeros(n, H, I, dtype=bf), "attn.q.weight": torch.zeros(H, H, dtype=bf),
         "mlp.gate.weight": torch.zeros(E, H, dtype=bf), "mlp.shared_expert.gate_proj.weight": torch.zeros(I, H, dtype=bf),
         "mlp.shared_expert.up_proj.weight": torch.zeros(I, H, dtype=bf), "norm": torch.zeros(H, dtype=torch.float32)}
    P = _FakePinned(t, list(range(n)))
    assert P.banks == {"gu": (E, 2 * I, H, g), "dn": (E, H, I, g)}
    plan = stream._UploadPlan(P)
    covered = torch.zeros(P.nbytes, dtype=torch.int32)
    for regions in plan.groups:
        for off, nb in regions:
            covered[off:off + nb] += 1
    inside = torch.zeros(P.nbytes, dtype=torch.bool)
    for off, _, _, nb in P.meta.values():
        inside[off:off + nb] = True
    assert bool((covered[inside] == 1).all()) and int(covered.max()) == 1
    kinds = [a[0] if a else None for a in plan.after]
    nch = -(-E // stream.BANK_CHUNK)
    assert kinds == ["bank"] * (2 * nch) + ["sel", None]
    for which in ("gu", "dn"):
        chunks = [a[2:] for a in plan.after if a and a[0] == "bank" and a[1] == which]
        assert chunks == [(e0, min(E, e0 + stream.BANK_CHUNK)) for e0 in range(0, E, stream.BANK_CHUNK)]
    lib = _lib.load()
    want = {"gu.f.q": lib.smel_packed_bytes(_lib.PACK_Q4, E * 2 * I, H),
            "gu.t.sz": lib.smel_packed_t_bytes(_lib.PACK_SZ, E, 2 * I, H, g),
            "dn.f.sz": lib.smel_packed_bytes(_lib.PACK_SZ, E * H, I),
            "experts.sel.down.t": lib.smel_packed_t_bytes(_lib.PACK_BF16, n, H, I, 0)}
    for k, nb in want.items():
        assert plan.pack_at[k][1] == nb
    spans = sorted((o, o + nb) for o, nb in plan.pack_at.values())
    assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:])) and spans[-1][1] <= plan.pack_bytes
    assert all(o % ALIGN == 0 for o, _ in plan.pack_at.values()) and len(plan.pack_at) == 12
