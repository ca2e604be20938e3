"""Parity and determinism of the HIP path at the full sizes of BASELINE.json's workloads C2-C5, each built exactly as
bench.py builds the step it times (bench.build_qwen_layer, build_gemma_block, gemma_block, c5_microbatches), so the
tile lists, k-loops, partial tiles and hot experts the bench measures are the ones checked here.

Bar: bf16 outputs and gradients against the fp32 oracle on the same inputs, with the
kernels' routing forced into the oracle as the reference's own tests force routing (tests/helpers.py:89-106):
||d|| / ||ref|| <= 2e-2, max|d| <= 2e-2 max|ref| and cosine >= 0.9999; bitwise equality over repeated runs. The
measured errors are printed next to the bar (pytest -s shows them).
"""
import pytest
import torch

import bench
from helpers import LORA_NAMES, assert_close_bf16
from oracle import moe_ref as R

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]
DEV = torch.device("cuda:0")


def _say(msg):
    print(msg, flush=True)


def _check(out, ref, name):
    e, m, c = assert_close_bf16(out.detach().float().cpu(), ref, name)
    _say(f"  {name:>10}: rel {e:.2e}  max {m:.2e}  cos {c:.7f}   (bar: 2e-2, 2e-2, 0.9999)")


def _lora_grads(lora):
    out = {}
    for tag, m in (("ex", lora.experts), ("sh", lora.shared)):
        if m is not None:
            for n in LORA_NAMES:
                out[f"{tag}_{n}"] = getattr(m, n).grad.detach().clone()
    return out


def _zero_grads(*mods):
    for m in mods:
        if m is not None:
            for p in m.parameters():
                p.grad = None


def _qwen_step(x, W, ex, lora, gy, K):
    """One fwd+bwd of the layer as bench.py's c3 / c5 step runs it; returns (y, dx, LoRA grads, topi)."""
    from smel.moe import moe_forward
    xg = x.clone().requires_grad_(True)
    seen = {}
    y = moe_forward(xg, W, ex, K, lora, stats=lambda p, v, i: seen.update(i=i.clone()))
    y.backward(gy)
    return y.detach(), xg.grad.detach(), _lora_grads(lora), seen["i"]


def test_c2_forward_full():
    """C2: the Qwen3.6-shaped layer forward, all 256 experts int4, shared expert, no LoRA (bench.py --workload c2)."""
    from smel.moe import moe_forward
    cfg = bench.QWEN
    _say("C2 full: T=4092 H=2048 E=256 I=512 K=8, all int4")
    x, W, ex, lora, gy = bench.build_qwen_layer(DEV, cfg, n_sel=0, lora=False)
    seen = {}
    with torch.no_grad():
        y = moe_forward(x, W, ex, cfg["K"], None, stats=lambda p, v, i: seen.update(i=i.clone()))
    torch.cuda.synchronize()
    ol = R.OracleLayer.from_api(W, ex, None)
    with torch.no_grad():
        yr = R.moe_forward(x.cpu(), ol, cfg["K"], forced_topi=seen["i"].cpu(), dtype=torch.float32)
    _check(y, yr, "y")


def test_c3_fwd_bwd_full():
    """C3 (the bench's default line): fwd+bwd with 12 bf16 + LoRA r16 experts and the shared LoRA: y, dX (incl. the
    router path) and all twelve LoRA gradients."""
    cfg = bench.QWEN
    _say("C3 full: T=4092 H=2048 E=256 I=512 K=8, 12 selected + LoRA r16, shared + LoRA r16")
    x, W, ex, lora, gy = bench.build_qwen_layer(DEV, cfg)
    y, dx, grads, topi = _qwen_step(x, W, ex, lora, gy, cfg["K"])
    torch.cuda.synchronize()
    ol = R.OracleLayer.from_api(W, ex, lora)
    yr, dxr, gr = R.moe_forward_backward(x.cpu(), ol, cfg["K"], gy.cpu(), forced_topi=topi.cpu(),
                                         dtype=torch.float32)
    _check(y, yr, "y")
    _check(dx, dxr, "dx")
    assert set(gr) == set(grads) and len(gr) == 12
    for k in sorted(gr):
        _check(grads[k], gr[k], k)


def test_c4_gemma_block_full():
    """C4: the Gemma-4-style block from the attention output on (six norms, route_gemma4, 128 GELU experts of I=704
    with 12 selected + LoRA, dense GeGLU 2112 + LoRA, residual adds, layer scalar): out, dh, da, all LoRA grads."""
    cfg = bench.GEMMA
    _say("C4 full: T=4096 H=2816 E=128 I=704 K=8, dense GeGLU 2112, 6 norms")
    h, a, W, ex, lora, gy = bench.build_gemma_block(DEV, cfg)
    hg, ag = h.clone().requires_grad_(True), a.clone().requires_grad_(True)
    seen = {}
    out = bench.gemma_block(hg, ag, W, ex, lora, cfg["K"], stats=lambda p, v, i: seen.update(i=i.clone()))
    out.backward(gy)
    torch.cuda.synchronize()
    grads = _lora_grads(lora)
    ol = R.OracleLayer.from_api(W, ex, lora, router_key="router.proj.weight")
    Wc = {k: v.detach().cpu() for k, v in W.items()}
    yr, dhr, dar, gr = R.gemma4_block_forward_backward(h.cpu(), a.cpu(), Wc, ol, cfg["K"], 1e-6, gy.cpu(),
                                                       forced_topi=seen["i"].cpu(), dtype=torch.float32)
    _check(out, yr, "out")
    _check(hg.grad, dhr, "dh")
    _check(ag.grad, dar, "da")
    assert set(gr) == set(grads) and len(gr) == 12
    for k in sorted(gr):
        _check(grads[k], gr[k], k)


def _c5_layer():
    cfg = dict(bench.QWEN, T=4096)
    return cfg, bench.build_qwen_layer(DEV, cfg, zipf=bench.C5_BIAS)


def test_c5_microbatch_full():
    """C5: one 4096-token micro-batch of the Zipf(1.2)-biased step, the 12 most popular experts selected: hot experts
    of more than 2000 rows (sixteen 128-row tiles), cold experts with none; y, dX and all LoRA grads."""
    cfg, (x, W, ex, lora, gy) = _c5_layer()
    _say("C5 micro-batch full: T=4096, Zipf-biased routing")
    y, dx, grads, topi = _qwen_step(x, W, ex, lora, gy, cfg["K"])
    torch.cuda.synchronize()
    counts = torch.bincount(topi.reshape(-1).cpu(), minlength=cfg["E"])
    _say(f"  rows per expert: max {int(counts.max())}, empty experts {int((counts == 0).sum())}")
    assert int(counts.max()) > 2000
    ol = R.OracleLayer.from_api(W, ex, lora)
    yr, dxr, gr = R.moe_forward_backward(x.cpu(), ol, cfg["K"], gy.cpu(), forced_topi=topi.cpu(),
                                         dtype=torch.float32)
    _check(y, yr, "y")
    _check(dx, dxr, "dx")
    for k in sorted(gr):
        _check(grads[k], gr[k], k)


def test_c5_step_bitwise_repeatable():
    """The whole C5 step (8 micro-batches of 4096 tokens, LoRA gradients accumulated over them, as bench.py times it)
    three times: every output, every dX and the accumulated gradients are bitwise equal."""
    from smel.moe import moe_forward
    cfg, (x, W, ex, lora, gy) = _c5_layer()
    xs, gys = bench.c5_microbatches(x, gy, 8, DEV)
    _say("C5 step x3: 8 x 4096 tokens")
    runs = []
    for _ in range(3):
        _zero_grads(lora)
        ys, dxs = [], []
        for xi, gi in zip(xs, gys):
            xg = xi.clone().requires_grad_(True)
            y = moe_forward(xg, W, ex, cfg["K"], lora)
            y.backward(gi)
            ys.append(y.detach())
            dxs.append(xg.grad.detach())
        runs.append((torch.stack(ys), torch.stack(dxs), _lora_grads(lora)))
    torch.cuda.synchronize()
    for r in runs[1:]:
        assert torch.equal(r[0].view(torch.int16), runs[0][0].view(torch.int16))
        assert torch.equal(r[1].view(torch.int16), runs[0][1].view(torch.int16))
        for k in runs[0][2]:
            assert torch.equal(r[2][k], runs[0][2][k]), k
