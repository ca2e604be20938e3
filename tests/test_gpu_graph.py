"""The fused MoE layer step (forward + backward) captured in a HIP graph and replayed gives bit-identical outputs and
gradients to eager execution, on every replay, with eager work and synchronizations between the replays."""
import pytest
import torch

from helpers import to_device_layer

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_graph_replay_matches_eager():
    from oracle import moe_ref as R
    from smel.moe import moe_forward
    print("graph replay of the fused layer (T=300, E=16, shared, LoRA)", flush=True)
    x, ol = R.make_layer(T=300, H=256, E=16, I=128, K=4, n_sel=3, r=8, alpha=16.0, shared_inter=128, group=64,
                         down_group=64, int4=True, seed=5, lora_b_std=0.02, dtype=torch.float32)
    W, ex, lora = to_device_layer(ol, DEV)
    x = x.to(DEV, torch.bfloat16)
    gy = (torch.randn(x.shape, generator=torch.Generator().manual_seed(1)) * 1e-2).to(DEV, torch.bfloat16)
    xg = x.clone().requires_grad_(True)
    params = list(lora.parameters())

    def step():
        xg.grad = None
        for p in params:
            p.grad = None
        y = moe_forward(xg, W, ex, 4, lora)
        y.backward(gy)
        return y

    def snapshot(y):
        return [y.detach().clone(), xg.grad.clone()] + [p.grad.clone() for p in params]

    ref = snapshot(step())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y_static = step()
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        got = snapshot(y_static)
        for a, b in zip(got, ref):
            assert torch.equal(a, b), f"replay {rep} differs from eager"
        # eager work between replays (the graph's buffers must not depend on it)
        eager = snapshot(step())
        torch.cuda.synchronize()
        for a, b in zip(eager, ref):
            assert torch.equal(a, b)
