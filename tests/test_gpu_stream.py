"""Layer streaming (smel.stream over include/smel_stream.h) on the GPU: layers staged from pinned host memory through
two device slots (copies on two copy streams, packing on the first, event hand-over) give the same tensors bit for
bit and the same MoE layer forward and backward bit for bit as the same layer built from resident device tensors
(the reference's build_layer path, smel/stream.py:16-36), over a sequence that evicts and re-stages layers while the
previous one is still computing."""
import pytest
import torch

pytestmark = pytest.mark.gpu
H, E, I, K, T = 256, 16, 128, 4, 256


@pytest.fixture(scope="module")
def mods():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from smel import moe, pack, stream
    return moe, pack, stream


def make_layer(pack, seed):
    """One packed layer (pack_layer's format, on the host) with two selected experts."""
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(seed)
    rn = lambda *s: (torch.randn(*s, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    gu, dn = rn(E, 2 * I, H), rn(E, H, I)
    sel = [1, 5 + seed % 3]
    t = {"mlp.experts.gate_up_proj": gu, "mlp.experts.down_proj": dn, "mlp.gate.weight": rn(E, H),
         "mlp.shared_expert.gate_proj.weight": rn(I, H), "mlp.shared_expert.up_proj.weight": rn(I, H),
         "mlp.shared_expert.down_proj.weight": rn(H, I), "mlp.shared_expert_gate.weight": rn(1, H),
         "self_attn.q_norm.weight": rn(64)}
    return {k: v.cpu() for k, v in pack.pack_layer(t, sel, 64).items()}


def run(moe, LW, x, gy):
    xg = x.clone().requires_grad_(True)
    y = moe.moe_forward(xg, LW.W, LW.experts, K)
    y.backward(gy)
    return y.detach(), xg.grad


def test_staged_layers_match_resident(mods):
    moe, pack, stream = mods
    layers = {l: make_layer(pack, l) for l in range(3)}
    resident = {}
    for l, t in layers.items():
        dt = {k: v.cuda() for k, v in t.items()}
        resident[l] = stream.build_layer(l, "linear_attention", dt, [int(i) for i in t["experts.sel.ids"]])
    g = torch.Generator(device="cuda").manual_seed(9)
    x = torch.randn(T, H, generator=g, device="cuda").to(torch.bfloat16)
    gy = (torch.randn(T, H, generator=g, device="cuda") * 1e-3).to(torch.bfloat16)
    want = {l: run(moe, LW, x, gy) for l, LW in resident.items()}

    src = stream.PinnedSource(layers, max_on_gpu=2)
    order = [0, 1, 2, 0, 2, 1, 1]
    for i, l in enumerate(order):
        print(f"stage step {i}: layer {l}", flush=True)
        LW = src.get(l)
        if i + 1 < len(order):
            src.prefetch(order[i + 1])        # evicts the other slot while layer l computes below
        for k, v in layers[l].items():
            if k != "experts.sel.ids":
                got = LW.W.get(k)
                if got is None:
                    got = {"experts.sel.gate_up": LW.experts.sel_gate_up, "experts.sel.down": LW.experts.sel_down}.get(k)
                if got is None:
                    which, part = k.split(".")[1:3]
                    got = (LW.experts.frozen.gu if which == "gate_up" else LW.experts.frozen.dn)[part]
                assert torch.equal(got.cpu(), v), (l, k)
        y, dx = run(moe, LW, x, gy)
        assert torch.equal(y, want[l][0]) and torch.equal(dx, want[l][1]), f"layer {l} at step {i}"
    gu = LW.W["mlp.shared_expert.gate_up_proj.weight"]
    assert gu.data_ptr() == LW.W["mlp.shared_expert.gate_proj.weight"].data_ptr()   # a view, no concatenation
    # uploads: 0, 1, 2 (evicts 0), 0 (evicts 1), 1 (evicts 0); layer 2 is still staged when prefetched again
    assert src.stats["loads"] == 5 and src.stats["bytes"] > 0
    src.close()


def test_dict_source(mods):
    _, _, stream = mods
    src = stream.DictSource({3: "layer"})
    src.prefetch(3)
    assert src.get(3) == "layer"
    src.close()


class _Ckpt:
    """The reference's Checkpoint interface (smel/model_io.py:220-252) over in-memory bf16 layers: layer(l) with
    layer-relative names and fused experts, full_name(l, short), get_rows(name, ids) and dims."""

    def __init__(self, layers, dims):
        self.layers, self.dims = layers, dims

    def layer(self, l):
        return dict(self.layers[l])

    def full_name(self, l, short):
        return f"model.layers.{l}.{short}"

    def get_rows(self, name, ids):
        _, _, l, short = name.split(".", 3)
        return self.layers[int(l)][short][list(ids)].clone()


def _checkpoint(nl=3):
    from types import SimpleNamespace
    g = torch.Generator().manual_seed(21)
    rn = lambda *s: (torch.randn(*s, generator=g) * 0.02).to(torch.bfloat16)
    layers = {l: {"mlp.experts.gate_up_proj": rn(E, 2 * I, H), "mlp.experts.down_proj": rn(E, H, I),
                  "mlp.gate.weight": rn(E, H), "mlp.shared_expert.gate_proj.weight": rn(I, H),
                  "mlp.shared_expert.up_proj.weight": rn(I, H), "mlp.shared_expert.down_proj.weight": rn(H, I),
                  "mlp.shared_expert_gate.weight": rn(1, H), "linear_attn.A_log": torch.randn(8, generator=g),
                  "input_layernorm.weight": torch.ones(H)} for l in range(nl)}
    return _Ckpt(layers, SimpleNamespace(layer_types=["linear_attention"] * nl, act="silu"))


def _inputs():
    g = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn(T, H, generator=g, device="cuda").to(torch.bfloat16)
    return x, (torch.randn(T, H, generator=g, device="cuda") * 1e-3).to(torch.bfloat16)


def _outputs(moe, src, layers, x, gy):
    out = {}
    for i, l in enumerate(layers):
        LW = src.get(l)
        if i + 1 < len(layers):
            src.prefetch(layers[i + 1])
        out[l] = run(moe, LW, x, gy) + (None if LW.experts.sel_ids is None else LW.experts.sel_ids.tolist(),)
    return out


@pytest.mark.parametrize("pin", [False, True])
def test_packed_source_matches_checkpoint_source(mods, tmp_path, pin):
    """Packed files written by pack_layer, streamed by PackedSource, give the same layers as CheckpointSource packing
    on the fly (the reference's test_packed_source_matches_dict, tests/test_stream_ckpt.py:45-66); the same layers
    with no selected experts differ."""
    moe, pack, stream = mods
    from safetensors.torch import save_file
    ck = _checkpoint()
    layers = [0, 1, 2]
    sel = {l: [l, l + 5] for l in layers}
    for l in layers:
        save_file(pack.pack_layer(ck.layer(l), sel[l], 64), str(tmp_path / f"layer_{l:02d}.safetensors"))
    x, gy = _inputs()
    print(f"packed source pin={pin}", flush=True)
    src_ck = stream.CheckpointSource(ck, "cuda", selection=sel, frozen="int4")
    want = _outputs(moe, src_ck, layers, x, gy)
    src = stream.PackedSource(str(tmp_path), ck.dims, layers, "cuda", pin=pin)
    got = _outputs(moe, src, layers, x, gy)
    allq = stream.CheckpointSource(ck, "cuda", selection={}, frozen="int4")
    plain = _outputs(moe, allq, layers, x, gy)
    for l in layers:
        assert got[l][2] == sel[l] and want[l][2] == sel[l] and plain[l][2] is None
        assert torch.equal(got[l][0], want[l][0]) and torch.equal(got[l][1], want[l][1]), l
        assert not torch.equal(plain[l][0], want[l][0])
    for s in (src_ck, src, allq):
        s.close()


def test_packed_source_reselection(mods, tmp_path):
    """A packed block re-selected from the original checkpoint (only the new experts' bf16 rows are read) equals the
    block packed with that selection in the first place; a layer left out of the new selection has none."""
    moe, pack, stream = mods
    from safetensors.torch import save_file
    ck = _checkpoint()
    layers = [0, 1, 2]
    for l in layers:
        save_file(pack.pack_layer(ck.layer(l), [1, 2], 64), str(tmp_path / f"layer_{l:02d}.safetensors"))
    new = {0: [7, 3, 12], 2: [4]}
    x, gy = _inputs()
    src = stream.PackedSource(str(tmp_path), ck.dims, layers, "cuda", selection=new, ckpt=ck)
    got = _outputs(moe, src, layers, x, gy)
    ref = stream.CheckpointSource(ck, "cuda", selection=new, frozen="int4")
    want = _outputs(moe, ref, layers, x, gy)
    for l in layers:
        assert got[l][2] == new.get(l) and want[l][2] == new.get(l)
        assert torch.equal(got[l][0], want[l][0]) and torch.equal(got[l][1], want[l][1]), l
    with pytest.raises(ValueError):
        stream.PackedSource(str(tmp_path), ck.dims, layers, "cuda", selection=new)
    src.close()
    ref.close()


def test_checkpoint_source_bf16(mods):
    """CheckpointSource with the bf16 bank: the same layers as build_layer on the checkpoint tensors moved to the
    device (dense tensors bf16, A_log kept fp32, selected experts copied from the bank)."""
    moe, _, stream = mods
    ck = _checkpoint()
    sel = {0: [2, 9], 1: []}
    src = stream.CheckpointSource(ck, "cuda", selection=sel)
    x, gy = _inputs()
    got = _outputs(moe, src, [0, 1, 2], x, gy)
    for l in (0, 1, 2):
        LW = stream.build_layer(l, "linear_attention", {k: v.cuda() for k, v in ck.layer(l).items()},
                                sel.get(l) or None)
        want = run(moe, LW, x, gy)
        assert got[l][2] == (sel.get(l) or None)
        assert torch.equal(got[l][0], want[0]) and torch.equal(got[l][1], want[1]), l
    LW = src.get(0)
    assert LW.W["linear_attn.A_log"].dtype == torch.float32 and LW.W["mlp.gate.weight"].dtype == torch.bfloat16
    src.close()
