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
