"""Benchmark of the MoE-layer hot path on one MI355X: forward with autograd + backward of the Qwen3.6-35B-A3B-shaped
MoE layer (T=4092, hidden 2048, 256 experts, top-8, expert intermediate 512, 244 frozen
int4 group-64 experts + 12 selected bf16 experts with LoRA r=16 alpha=32, shared expert 512 with LoRA r=16,
upstream grad ~N(0, 1e-3)). Synthetic data, random weights of that shape (weights ~N(0, 0.02), x ~N(0, 1)).

One JSON line on stdout: tokens/s of the whole layer step, the roofline of the dominant kernel (HIP-event timed
launches inside this run) and the CPU baseline (the oracle's restatement of the reference's CPU torch path, timed on
this host's cores on one full pass of the same layer).
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "smel-ft_amd")]

import torch  # noqa: E402

METRIC = json.load(open(os.path.join(ROOT, "BASELINE.json")))["metric"]
HBM_PEAK = 8.0e12            # B/s, MI355X
MFMA_BF16_PEAK = 2.5e15      # FLOP/s, MI355X dense bf16

C3 = dict(T=4092, H=2048, E=256, I=512, K=8, Is=512, r=16, alpha=32.0, n_sel=12, group=64)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_layer(device, cfg=C3, seed=0):
    """The C3 layer with the drop-in API's own types; the frozen bank is quantized on the GPU by smel.quant."""
    from smel.lora import ExpertsLoRA, LayerLoRA, MLPLoRA
    from smel.moe import Int4Experts, LayerExperts
    g = torch.Generator(device=device).manual_seed(seed)
    T, H, E, I, Is, r = cfg["T"], cfg["H"], cfg["E"], cfg["I"], cfg["Is"], cfg["r"]
    bf = torch.bfloat16

    def rnd(*s, std=0.02):
        return (torch.randn(*s, generator=g, device=device) * std).to(bf)

    x = torch.randn(T, H, generator=g, device=device).to(bf)
    W = {"mlp.gate.weight": rnd(E, H),
         "mlp.shared_expert.gate_proj.weight": rnd(Is, H), "mlp.shared_expert.up_proj.weight": rnd(Is, H),
         "mlp.shared_expert.down_proj.weight": rnd(H, Is), "mlp.shared_expert_gate.weight": rnd(1, H)}
    gu, dn = rnd(E, 2 * I, H), rnd(E, H, I)
    bank = Int4Experts.from_bf16(gu, dn, cfg["group"])
    sel = list(range(0, E, E // cfg["n_sel"]))[: cfg["n_sel"]]        # scripts/bench/bench_layer.py:70
    ex = LayerExperts(bank, sel, gu[sel].clone(), dn[sel].clone(), group=32)
    del gu, dn
    torch.manual_seed(seed)
    lora = LayerLoRA(ExpertsLoRA(sel, H, I, r, cfg["alpha"]), MLPLoRA(H, Is, r, cfg["alpha"])).to(device)
    gy = (torch.randn(T, H, generator=g, device=device) * 1e-3).to(bf)
    torch.cuda.synchronize()
    return x, W, ex, lora, gy


def gemm_flops(tag, cfg, S):
    """Algorithmic FLOPs of one launch of each grouped GEMM (routed + shared rows, LoRA at its real rank r)."""
    T, H, E, I, K, r = cfg["T"], cfg["H"], cfg["E"], cfg["I"], cfg["K"], cfg["r"]
    M = T * K + T          # routed slots + shared-expert rows
    Lr = S + T             # rows with LoRA (selected-expert slots + shared rows)
    return {"gemm_gu_fwd": 2 * M * H * 2 * I + 2 * Lr * r * 2 * I,
            "gemm_dn_fwd": 2 * M * I * H + 2 * Lr * r * H,
            "gemm_dn_bwd": 2 * M * H * I + 2 * Lr * r * I,
            "gemm_gu_bwd": 2 * M * 2 * I * H + 2 * Lr * 2 * r * H,
            "gemm_router_bwd": 2 * T * (E + 1) * H}.get(tag)


def cpu_baseline(x, W, ex, lora, gy, cfg):
    """The oracle (CPU restatement of the reference's CPU torch path, fp32) on one full pass of the same layer."""
    from oracle import moe_ref as R
    cores = min(16, os.cpu_count() or 1)
    torch.set_num_threads(cores)
    c = lambda t: t.detach().cpu()
    fz = {"gate_up": {k: c(v) for k, v in ex.frozen.gu.items()}, "down": {k: c(v) for k, v in ex.frozen.dn.items()}}
    names = ("A_gate", "B_gate", "A_up", "B_up", "A_down", "B_down")
    Is = cfg["Is"]
    ol = R.OracleLayer(gate_w=c(W["mlp.gate.weight"]), frozen=fz, int4=True, sel_ids=[int(e) for e in ex.sel_ids],
                       sel_gate_up=c(ex.sel_gate_up), sel_down=c(ex.sel_down),
                       ex_lora={n: c(getattr(lora.experts, n)) for n in names}, ex_scale=lora.experts.scale,
                       shared={"gate_up": torch.cat((c(W["mlp.shared_expert.gate_proj.weight"]),
                                                     c(W["mlp.shared_expert.up_proj.weight"]))),
                               "down": c(W["mlp.shared_expert.down_proj.weight"]),
                               "gate_w": c(W["mlp.shared_expert_gate.weight"])},
                       sh_lora={n: c(getattr(lora.shared, n)) for n in names}, sh_scale=lora.shared.scale,
                       deq_dtype=torch.bfloat16)
    assert ol.shared["down"].shape[1] == Is
    t0 = time.perf_counter()
    R.moe_forward_backward(c(x), ol, cfg["K"], c(gy), dtype=torch.float32)
    dt = time.perf_counter() - t0
    return {"value": cfg["T"] / dt, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"1 fwd+bwd pass of the full C3 layer (T={cfg['T']}), fp32, {dt:.1f} s, "
                      f"torch threads={cores}, cpu={_cpu_model()}"}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true", help="time eager launches only (no HIP graph replay)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the MoE hot path here runs on one MI355X and has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)
    from smel import _lib
    from smel.moe import moe_forward
    _lib.load()
    dev = torch.device("cuda:0")
    cfg = C3
    log("building the C3 layer (int4 quantization on the GPU) ...")
    x, W, ex, lora, gy = build_layer(dev, cfg)
    xg = x.clone().requires_grad_(True)
    params = list(lora.parameters())
    seen = {}

    def step(stats=None):
        xg.grad = None
        for p in params:
            p.grad = None
        y = moe_forward(xg, W, ex, cfg["K"], lora, stats=stats)
        y.backward(gy)

    step(stats=lambda p, v, i: seen.update(topi=i))
    sel = torch.zeros(cfg["E"], dtype=torch.bool, device=dev)
    sel[ex.sel_ids.to(dev)] = True
    S = int(sel[seen["topi"]].sum())
    log(f"slots routed to the selected experts: S={S} (S/T={S / cfg['T']:.3f})")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    eager_ms = dt / args.steps * 1e3
    log(f"eager step {eager_ms:.3f} ms, {cfg['T'] * args.steps / dt:.0f} tokens/s")
    mode = "eager"
    ms, tok_s = eager_ms, cfg["T"] * args.steps / dt
    if not args.eager:
        # The same step (forward + backward, every kernel) captured once in a HIP graph and replayed: this removes
        # the host-side launch gaps between the ~40 kernels of a step. Capture on a side stream of default priority
        # after a few warm-up steps there (allocator pools settle), as torch.cuda.graph expects.
        gs = torch.cuda.Stream()
        gs.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(gs):
            for _ in range(3):
                step()
        torch.cuda.current_stream().wait_stream(gs)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            graph.replay()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        mode = "hip_graph"
        ms, tok_s = dt / args.steps * 1e3, cfg["T"] * args.steps / dt
        log(f"graph step {ms:.3f} ms, {tok_s:.0f} tokens/s")
    # per-launch timing of every entry point (events on the launching stream), a few extra steps
    n_prof = max(5, min(20, args.steps))
    with _lib.timing() as tm:
        for _ in range(n_prof):
            step()
    torch.cuda.synchronize()
    res = tm.results()
    breakdown = {k: round(statistics.mean(v), 4) for k, v in sorted(res.items(), key=lambda kv: -sum(kv[1]))}
    log("per-launch ms:", json.dumps(breakdown))
    gemms = {k: v for k, v in breakdown.items() if gemm_flops(k, cfg, S)}
    dom = max(gemms, key=gemms.get)
    F = gemm_flops(dom, cfg, S)
    achieved = F / (gemms[dom] * 1e-3)
    roof = {"kernel": dom, "bound": "mfma", "achieved": round(achieved / 1e12, 2), "peak": MFMA_BF16_PEAK / 1e12,
            "unit": "TFLOP/s", "frac": round(achieved / MFMA_BF16_PEAK, 4), "traffic": None,
            "flops_per_launch": F, "avg_launch_ms": gemms[dom]}
    total_f = sum(gemm_flops(k, cfg, S) for k in gemms)
    out = {"metric": METRIC, "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "bf16", "data": "synthetic (random weights ~N(0,0.02), x ~N(0,1))",
           "config": {"workload": "C3: Qwen3.6-35B-A3B MoE layer fwd+bwd, T=4092, H=2048, E=256, I=512, top-8, "
                                  "244 int4 g64 frozen + 12 bf16 LoRA r16 experts, shared 512 + LoRA r16",
                      "tokens": cfg["T"], "selected_slots": S, "parallelism": "single GPU", "launch": mode},
           "eager_ms_per_step": round(eager_ms, 4),
           "roofline": roof,
           "gemm_tflops_all": round(total_f / (sum(gemms.values()) * 1e-3) / 1e12, 2),
           "breakdown_ms": breakdown}
    if not args.no_cpu_baseline:
        log("timing the CPU baseline (one full pass of the oracle) ...")
        out["cpu_baseline"] = cpu_baseline(x, W, ex, lora, gy, cfg)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
