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
