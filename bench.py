"""Benchmark of the MoE-layer hot path on one MI355X.

Default (the driver's line): forward with autograd + backward of the Qwen3.6-35B-A3B-shaped MoE layer (BASELINE.json
configs[2], "C3": T=4092, hidden 2048, 256 experts, top-8, expert intermediate 512, 244 frozen int4 group-64 experts
+ 12 selected bf16 experts with LoRA r=16 alpha=32, shared expert 512 with LoRA r=16, upstream grad ~N(0, 1e-3)).
Synthetic data, random weights of that shape (weights ~N(0, 0.02), x ~N(0, 1)).

Other workloads of BASELINE.json (``--workload``), each printing one JSON line of its own:
  c2  forward only (no autograd) of the same layer with all 256 experts frozen int4 and no LoRA;
  c4  Gemma-4-26B-A4B-style MoE block fwd+bwd: the Gemma 4 layer from the attention output on
      (smel/layer_runner.py:243-262): six RMSNorms, route_gemma4 on the residual stream, 128 GELU-tanh experts
      (I=704, 12 selected bf16 + LoRA r16, the rest int4), the dense GeGLU MLP (2112) with LoRA r16, the residual
      adds and the layer scalar, T=4096 as 8 packed sequences (the block is token-wise: cu_seqlens change nothing);
  c5  the Qwen layer under skewed routing: T=32768 as 8 micro-batches of 4096, router biased to a
      Zipf(1.2) expert popularity (realised top-12 gate-mass share reported), the 12 most popular experts selected.
  stream  the C3 layer with its weights (int4 bank, selected experts, router, shared expert) staged from pinned host
      memory into two device slots per layer (include/smel_stream.h): host -> device bandwidth with one and two copy
      streams, and the layer-major loop over 4 layer ids (each layer's upload and packing overlapping the previous
      layer's fwd+bwd) against the resident layer;
  quant  the GPU int4 quantizer (the pack stage's producer of the on-disk format) on the C2 bank: 256 experts,
      gate_up [256, 1024, 2048] and down [256, 2048, 512] bf16, group 64, the reference's five clip factors;
  ce  the single-pass chunked cross-entropy (loss + dh) over a Qwen3.6-sized head: 4092 tokens, hidden 2048, vocabulary
      248320, bf16, token chunk 1024, vocabulary chunk 32768;
  norms  the RMSNorm family around the block (include/smel_norm.h), forward + backward at the Qwen3.6 block's
      shapes for T=4092: input norm and residual add + post-attention norm [T, 2048], q / k head norms
      [T, 16 | 2, 256] (q a strided half of q_proj's output), the gated DeltaNet output norm [T * 32, 128];
  c3f32  the C3 layer with float32 activations and weights (the reference's fp32 models) on the fp32 kernels
      (include/smel_f32.h), eager fwd+bwd, roofline against the dense fp32 MFMA peak;
  peaks  the achievable MFMA rate and HBM bandwidth of this GPU by kernels that do nothing else
      (include/smel_probe.h), and hipBLASLt's bf16 GEMM for comparison.

Every line carries tokens/s of the whole step, the roofline of the dominant kernel (HIP-event timed launches inside
this run: algorithmic FLOPs and bytes per launch against MI355X's dense bf16 MFMA and HBM peaks, the binding one
reported; beside it the fraction of the achievable peak measured by the probes of ``--workload peaks``, its HBM
traffic and MFMA-busy share from the committed rocprofv3 --pmc summaries) and, for C3 and C2, the CPU baseline (the oracle's restatement of the reference's CPU torch path, timed on this
host's cores on one full pass of the same layer).
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

QWEN = dict(T=4092, H=2048, E=256, I=512, K=8, Is=512, r=16, alpha=32.0, n_sel=12, group=64, act="silu")
GEMMA = dict(T=4096, H=2816, E=128, I=704, K=8, Is=2112, r=16, alpha=32.0, n_sel=12, group=64, act="gelu_tanh")
C5_BIAS = 0.45               # Zipf bias scale giving a ~50% top-12 gate-mass share (calibrated on the GPU)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------------------------------------- layer builders


def _rnd(g, device, *s, std=0.02):
    return (torch.randn(*s, generator=g, device=device) * std).to(torch.bfloat16)


def _randomize_lora_b(lora, g, std=0.02):
    """LoRA B factors ~N(0, std) instead of the init's zeros, so that every LoRA product and gradient of the step is
    non-trivial (dA is exactly 0 while B = 0); the work is the same either way."""
    with torch.no_grad():
        for m in (lora.experts, lora.shared):
            if m is not None:
                for n in ("B_gate", "B_up", "B_down"):
                    p = getattr(m, n)
                    p.copy_(torch.randn(p.shape, generator=g, device=p.device) * std)


def build_qwen_layer(device, cfg=QWEN, seed=0, n_sel=None, lora=True, zipf=None):
    """The Qwen layer with the drop-in API's own types; the frozen bank is quantized on the GPU by smel.quant.
    ``zipf`` = bias scale c: expert e (in a random popularity order) gets logit bias -1.2 c ln(rank), injected
    through the API's inputs: x has a unit mean component and router row e adds bias_e / H to every entry (rows
    centred first, so the bias is the only mean term)."""
    from smel.lora import ExpertsLoRA, LayerLoRA, MLPLoRA
    from smel.moe import Int4Experts, LayerExperts
    g = torch.Generator(device=device).manual_seed(seed)
    T, H, E, I, Is, r = cfg["T"], cfg["H"], cfg["E"], cfg["I"], cfg["Is"], cfg["r"]
    n_sel = cfg["n_sel"] if n_sel is None else n_sel
    x = torch.randn(T, H, generator=g, device=device)
    gate = torch.randn(E, H, generator=g, device=device) * 0.02
    popular = None
    if zipf is not None:
        perm = torch.randperm(E, generator=torch.Generator().manual_seed(seed + 1))
        rank = torch.empty(E, dtype=torch.long)
        rank[perm] = torch.arange(E)
        bias = -1.2 * zipf * torch.log(rank.double() + 1.0)
        gate = gate - gate.mean(1, keepdim=True) + (bias / H).float().to(device)[:, None]
        x = x + 1.0
        popular = perm[:n_sel].tolist()
    x = x.to(torch.bfloat16)
    W = {"mlp.gate.weight": gate.to(torch.bfloat16),
         "mlp.shared_expert.gate_proj.weight": _rnd(g, device, Is, H),
         "mlp.shared_expert.up_proj.weight": _rnd(g, device, Is, H),
         "mlp.shared_expert.down_proj.weight": _rnd(g, device, H, Is),
         "mlp.shared_expert_gate.weight": _rnd(g, device, 1, H)}
    gu, dn = _rnd(g, device, E, 2 * I, H), _rnd(g, device, E, H, I)
    bank = Int4Experts.from_bf16(gu, dn, cfg["group"])
    if n_sel:
        sel = popular if popular is not None else list(range(0, E, E // n_sel))[:n_sel]   # bench_layer.py:70
        ex = LayerExperts(bank, sel, gu[sel].clone(), dn[sel].clone(), group=32, act=cfg["act"])
    else:
        sel = []
        ex = LayerExperts(bank, group=32, act=cfg["act"])
    del gu, dn
    torch.manual_seed(seed)
    lo = None
    if lora:
        lo = LayerLoRA(ExpertsLoRA(sel, H, I, r, cfg["alpha"]) if sel else None,
                       MLPLoRA(H, Is, r, cfg["alpha"])).to(device)
        _randomize_lora_b(lo, g)
    gy = (torch.randn(T, H, generator=g, device=device) * 1e-3).to(torch.bfloat16)
    torch.cuda.synchronize()
    return x, W, ex, lo, gy


GEMMA_NORMS = ("post_attention_layernorm", "pre_feedforward_layernorm", "post_feedforward_layernorm_1",
               "pre_feedforward_layernorm_2", "post_feedforward_layernorm_2", "post_feedforward_layernorm")


def build_gemma_block(device, cfg=GEMMA, seed=0):
    """The Gemma-4-style block's inputs and weights: residual stream h and attention output a, the six norm weights
    (~1 + N(0, 0.2)) and the layer scalar, router tensors as smel/tiny.py:74-77 draws them, 128 experts (12 selected
    bf16 + LoRA, the rest int4), dense GeGLU MLP + LoRA. Returns (h, a, W, LayerExperts, LayerLoRA, upstream grad)."""
    from smel.lora import ExpertsLoRA, LayerLoRA, MLPLoRA
    from smel.moe import Int4Experts, LayerExperts
    g = torch.Generator(device=device).manual_seed(seed)
    T, H, E, I, Is, r = cfg["T"], cfg["H"], cfg["E"], cfg["I"], cfg["Is"], cfg["r"]
    h = (torch.randn(T, H, generator=g, device=device) * 3.0).to(torch.bfloat16)
    a = torch.randn(T, H, generator=g, device=device).to(torch.bfloat16)
    W = {f"{n}.weight": (1.0 + 0.2 * torch.randn(H, generator=g, device=device)).to(torch.bfloat16)
         for n in GEMMA_NORMS}
    W.update({"router.scale": (1.0 + 0.2 * torch.randn(H, generator=g, device=device)).to(torch.bfloat16),
              "router.proj.weight": _rnd(g, device, E, H),
              "router.per_expert_scale": (0.5 + torch.rand(E, generator=g, device=device)).to(torch.bfloat16),
              "mlp.gate_up_proj.weight": _rnd(g, device, 2 * Is, H), "mlp.down_proj.weight": _rnd(g, device, H, Is),
              "layer_scalar": torch.full((1,), 0.8, device=device).to(torch.bfloat16)})
    W["mlp.gate_proj.weight"] = W["mlp.gate_up_proj.weight"][:Is]
    W["mlp.up_proj.weight"] = W["mlp.gate_up_proj.weight"][Is:]
    gu, dn = _rnd(g, device, E, 2 * I, H), _rnd(g, device, E, H, I)
    bank = Int4Experts.from_bf16(gu, dn, cfg["group"])
    sel = list(range(0, E, E // cfg["n_sel"]))[: cfg["n_sel"]]
    ex = LayerExperts(bank, sel, gu[sel].clone(), dn[sel].clone(), group=32, act=cfg["act"])
    del gu, dn
    torch.manual_seed(seed)
    lora = LayerLoRA(ExpertsLoRA(sel, H, I, r, cfg["alpha"]), MLPLoRA(H, Is, r, cfg["alpha"])).to(device)
    _randomize_lora_b(lora, g)
    gy = (torch.randn(T, H, generator=g, device=device) * 1e-3).to(torch.bfloat16)
    torch.cuda.synchronize()
    return h, a, W, ex, lora, gy


def gemma_block(h, a, W, ex, lora, top_k, eps=1e-6, stats=None):
    """The Gemma 4 layer from the attention output on, through the drop-in API (smel/layer_runner.py:243-262: norm
    and MoE calls in the reference's order): every norm and MoE step is a HIP launch; the residual adds and the
    layer-scalar product are torch element-wise ops."""
    from smel.moe import mlp_lora, route_gemma4, routed_experts
    from smel.norm import add_rmsnorm, rmsnorm
    nw = lambda n: W[n + ".weight"]
    h2, xm = add_rmsnorm(h, rmsnorm(a, nw("post_attention_layernorm"), eps, False), nw("pre_feedforward_layernorm"),
                         eps, False)
    m = mlp_lora(xm, W["mlp.gate_proj.weight"], W["mlp.up_proj.weight"], W["mlp.down_proj.weight"], lora.shared,
                 ex.act, W["mlp.gate_up_proj.weight"])
    m = rmsnorm(m, nw("post_feedforward_layernorm_1"), eps, False)
    probs, topv, topi = route_gemma4(h2, W, top_k, eps)
    if stats is not None:
        stats(probs, topv, topi)
    e = routed_experts(rmsnorm(h2, nw("pre_feedforward_layernorm_2"), eps, False), topv, topi, ex, lora.experts)
    e = rmsnorm(e, nw("post_feedforward_layernorm_2"), eps, False)
    _, y = add_rmsnorm(m, e, nw("post_feedforward_layernorm"), eps, False)
    return (h2 + y) * W["layer_scalar"]


def c5_microbatches(x, gy, n, device):
    """The C5 step's n micro-batches of the same layer: the first is (x, gy), the others x + 0.5 N(0, 1) with fresh
    upstream gradients (the same Zipf-biased router sees each)."""
    xs, gys = [x], [gy]
    g = torch.Generator(device=device).manual_seed(7)
    for _ in range(n - 1):
        xs.append((x.float() + 0.5 * torch.randn(x.shape, generator=g, device=device)).to(torch.bfloat16))
        gys.append((torch.randn(gy.shape, generator=g, device=device) * 1e-3).to(torch.bfloat16))
    return xs, gys


# ------------------------------------------------------------------------------------------ algorithmic work model


def kernel_work(tag, c, S):
    """(algorithmic FLOPs, algorithmic HBM bytes) of one launch of a kernel, from the layer's shape ``c`` and the
    number S of slots routed to selected experts. Bytes = every operand read once and every result written once:
    frozen int4 experts (q + bf16 scale/zero, the reference's format) except the selected ones, selected / shared
    bf16 weights, activations
    (the gathered token rows counted once per token), the LoRA K-extension rows, the saved pre-activations and (down
    backward) the saved activation."""
    T, H, E, I, K, r = c["T"], c["H"], c["E"], c["I"], c["K"], c["r"]
    g = c["group"]
    n_sel = c.get("n_sel_used", c["n_sel"])
    Msh = T if c.get("fused_shared") else 0
    M = T * K + Msh
    Lr = S + Msh
    nfz = E - n_sel
    # int4 weights counted in the reference's format (smel/quant.py:24-44: two nibbles per byte, a bf16 scale and a
    # bf16 zero per group = 4 B), whatever layout a kernel reads them in
    def bank(nq, ngroups, nbf):
        return nfz * (nq // 2 + ngroups * 4) + n_sel * nbf * 2 + (nbf * 2 if Msh else 0)
    gu_w = gu_wt = bank(2 * I * H, 2 * I * (H // g), 2 * I * H)
    dn_w = dn_wt = bank(H * I, H * (I // g), H * I)
    ext = M * 32 * 2 if (Lr and r) else 0
    nblk = -(-I // 128)
    Epad = -(-(E + (1 if Msh else 0)) // 32) * 32
    Is = c.get("Is", I)
    w = {"gemm_gu_fwd": (2 * M * H * 2 * I + 2 * Lr * r * 2 * I, gu_w + T * H * 2 + ext + M * I * 2 + M * 2 * I * 2),
         "gemm_dn_fwd": (2 * M * I * H + 2 * Lr * r * H, dn_w + M * I * 2 + ext + M * H * 2),
         "gemm_dn_bwd": (2 * M * H * I + 2 * Lr * r * I,
                         dn_wt + T * H * 2 + M * 2 * I * 2 + M * I * 2 + ext + M * 2 * I * 2 + M * nblk * 4),
         "gemm_gu_bwd": (2 * M * 2 * I * H + 2 * Lr * 2 * r * H, gu_wt + M * 2 * I * 2 + ext + M * H * 2),
         "gemm_router_bwd": (2 * T * Epad * H, T * Epad * 2 + Epad * H * 2 + T * H * 2),
         "gemm_mlp_gu_fwd": (2 * T * H * 2 * Is + 2 * T * r * 2 * Is,
                             2 * Is * H * 2 + T * H * 2 + T * 64 + T * Is * 2 + T * 2 * Is * 2),
         "gemm_mlp_dn_fwd": (2 * T * Is * H + 2 * T * r * H, H * Is * 2 + T * Is * 2 + T * 64 + T * H * 2),
         "gemm_mlp_dn_bwd": (2 * T * H * Is + 2 * T * r * Is, H * Is * 2 + T * H * 2 + 2 * T * 2 * Is * 2 + T * 64),
         "gemm_mlp_gu_bwd": (2 * T * 2 * Is * H + 2 * T * 2 * r * H,
                             2 * Is * H * 2 + T * 2 * Is * 2 + T * 64 + T * H * 2),
         "smel_combine": (0, M * H * 2 + T * K * 2 + T * 4 + T * H * 2),
         "smel_dx_reduce": (0, M * H * 2 + 2 * T * H * 2)}
    return w.get(tag)


def roofline(breakdown, c, S, pmc=False):
    """The dominant (longest average launch) kernel with a work model: its roofline time max(F / P_mfma,
    B / BW_hbm) decides the bound; achieved = that kernel's F or B over its HIP-event-timed launch. pmc: the
    workload is the one the committed rocprofv3 --pmc summaries were taken on (C3), so its HBM traffic and MFMA-busy
    share are reported from them."""
    known = {k: v for k, v in breakdown.items() if kernel_work(k, c, S)}
    dom = max(known, key=known.get)
    F, B = kernel_work(dom, c, S)
    t = known[dom] * 1e-3
    if F / MFMA_BF16_PEAK >= B / HBM_PEAK:
        out = {"kernel": dom, "bound": "mfma", "achieved": round(F / t / 1e12, 2), "peak": MFMA_BF16_PEAK / 1e12,
               "unit": "TFLOP/s", "frac": round(F / t / MFMA_BF16_PEAK, 4)}
    else:
        out = {"kernel": dom, "bound": "hbm", "achieved": round(B / t / 1e9, 1), "peak": HBM_PEAK / 1e9,
               "unit": "GB/s", "frac": round(B / t / HBM_PEAK, 4)}
    out.update({"traffic": measured_traffic(dom) if pmc else None, "flops_per_launch": F, "bytes_per_launch": B,
                "avg_launch_ms": known[dom], "mfma_frac": round(F / t / MFMA_BF16_PEAK, 4),
                "hbm_frac": round(B / t / HBM_PEAK, 4)})
    pk = _profile("peaks.json")
    if pk:
        m = pk["measured"]
        ach = m["mfma_loop_tflops"] * 1e12 if out["bound"] == "mfma" else m["read_gbps"] * 1e9
        out.update({"achievable_peak": round(ach / (1e12 if out["bound"] == "mfma" else 1e9), 1),
                    "frac_of_achievable": round((F if out["bound"] == "mfma" else B) / t / ach, 4)})
    busy = (_profile("mfma.json") or {}).get("kernels", {}).get(dom) if pmc else None
    if busy:
        out["mfma_busy_pmc"] = busy["mfma_busy"]
    return out


def _profile(name):
    """A committed measurement summary from profiles/ (JSON), or None."""
    try:
        return json.load(open(os.path.join(ROOT, "profiles", name)))
    except (OSError, ValueError):
        return None


def measured_traffic(kernel_tag):
    """HBM bytes per launch of a kernel from the committed rocprofv3 --pmc summary (profiles/traffic.json: FETCH_SIZE
    and WRITE_SIZE per dispatch, scaled by the same counters on a copy of known size), or None if not measured."""
    d = _profile("traffic.json")
    if d is None:
        return None
    k = d.get("kernels", {}).get(kernel_tag)
    return None if k is None else k.get("hbm_bytes_per_launch")


# ---------------------------------------------------------------------------------------------------- timing


def time_step(step, steps, warmup, graph):
    """Eager timing of ``steps`` steps after ``warmup``, then (graph=True) the same step captured once in a HIP
    graph and replayed (removes the host launch gaps between the step's kernels). Returns (mode, ms, eager_ms)."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) / steps * 1e3
    log(f"eager step {eager_ms:.3f} ms")
    if not graph:
        return "eager", eager_ms, eager_ms
    # capture on a side stream of default priority after a few warm-up steps there (allocator pools settle)
    gs = torch.cuda.Stream()
    gs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(gs):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(gs)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        g.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    log(f"graph step {ms:.3f} ms")
    return "hip_graph", ms, eager_ms


def breakdown_of(step, n):
    """Per-launch milliseconds of every entry point over n extra eager steps, by HIP events on the launching stream:
    the median over its launches (a launch whose start event waited on the host, e.g. for an allocation, would pull
    a mean far from what a kernel trace shows). The side-stream forks of the step run on the main stream for this
    (launch order kept), so each event pair brackets one launch with nothing beside it: the launch's own duration.
    (With the forks on, a launch's start event also counts the wait for compute units that the forked kernels
    hold.)"""
    from smel import _lib
    from smel import moe
    forks, moe._SIDE_ON = moe._SIDE_ON, frozenset()
    try:
        with _lib.timing() as tm:
            for _ in range(n):
                step()
        torch.cuda.synchronize()
    finally:
        moe._SIDE_ON = forks
    res = tm.results()
    return {k: round(statistics.median(v), 4) for k, v in sorted(res.items(), key=lambda kv: -statistics.median(kv[1]))}


def emit(metric, tokens, args, timing, workload, extra_cfg, roof, breakdown, cpu=None, **extra):
    mode, ms, eager_ms = timing
    out = {"metric": metric, "value": round(tokens / ms * 1e3, 1), "unit": "tokens/s", "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic (random weights ~N(0,0.02), x ~N(0,1))",
           "config": {"workload": workload, "tokens": tokens, "parallelism": "single GPU", "launch": mode,
                      **extra_cfg},
           "eager_ms_per_step": round(eager_ms, 4), "roofline": roof, "breakdown_ms": breakdown,
           "cpu_baseline": cpu}
    out.update(extra)
    print(json.dumps(out), flush=True)


# ------------------------------------------------------------------------------------------------- workloads

QWEN_NAMES = {
    "c3": ("C3: Qwen3.6-35B-A3B MoE layer fwd+bwd, T=4092, H=2048, E=256, I=512, top-8, 244 int4 g64 frozen + 12 bf16 "
           "LoRA r16 experts, shared 512 + LoRA r16"),
    "c2": ("C2: Qwen3.6-35B-A3B MoE layer forward only, T=4092, H=2048, E=256, I=512, top-8, all 256 experts int4 "
           "g64, shared expert 512 (no LoRA)"),
    "c5": ("C5: Qwen3.6 MoE layer fwd+bwd under Zipf(1.2)-biased routing, T=32768 as 8 micro-batches of 4096, the 12 "
           "most popular experts bf16 + LoRA r16, shared 512 + LoRA r16")}
QWEN_METRICS = {"c2": "MoE layer forward tokens/s (Qwen3.6 shape, T=4092)",
                "c5": "MoE layer fwd+bwd tokens/s under Zipf-skewed routing (Qwen3.6 shape, 8 x 4096 tokens)"}


def run_qwen(args, dev, mode):
    """c3 (default): fwd+bwd with LoRA; c2: forward only, all experts int4, no LoRA; c5: c3 under Zipf routing,
    8 micro-batches of 4096 tokens per step."""
    from smel.moe import moe_forward
    cfg = dict(QWEN)
    fwd_only = mode == "c2"
    nmb = 1
    if mode == "c5":
        cfg["T"] = 4096
        nmb = 8
    log(f"building the {mode} layer (int4 quantization on the GPU) ...")
    x, W, ex, lora, gy = build_qwen_layer(dev, cfg, n_sel=0 if fwd_only else None, lora=not fwd_only,
                                          zipf=C5_BIAS if mode == "c5" else None)
    T = cfg["T"]
    xs, gys = c5_microbatches(x, gy, nmb, dev)   # nmb = 1: just (x, gy)
    xgs = [xi.clone().requires_grad_(not fwd_only) for xi in xs]
    params = list(lora.parameters()) if lora is not None else []
    seen = []

    def step(stats=None):
        if fwd_only:
            with torch.no_grad():
                for xi in xgs:
                    moe_forward(xi, W, ex, cfg["K"], None, stats=stats)
            return
        for p in params:
            p.grad = None
        for xi, gi in zip(xgs, gys):
            xi.grad = None
            moe_forward(xi, W, ex, cfg["K"], lora, stats=stats).backward(gi)

    step(stats=lambda p, v, i: seen.append((v.float(), i)))
    sel = torch.zeros(cfg["E"], dtype=torch.bool, device=dev)
    if ex.sel_ids is not None:
        sel[ex.sel_ids.to(dev)] = True
    S = int(sum(int(sel[i].sum()) for _, i in seen) / len(seen))
    extra = {}
    if mode == "c5":
        mass = torch.zeros(cfg["E"], dtype=torch.float64, device=dev)
        cnt = torch.zeros(cfg["E"], dtype=torch.float64, device=dev)
        for v, i in seen:
            mass.index_add_(0, i.reshape(-1), v.reshape(-1).double())
            cnt.index_add_(0, i.reshape(-1), torch.ones(i.numel(), dtype=torch.float64, device=dev))
        share = float(mass.sort(descending=True).values[:12].sum() / mass.sum())
        sel_share = float(mass[sel].sum() / mass.sum())
        extra = {"top12_gate_mass_share": round(share, 4), "selected_gate_mass_share": round(sel_share, 4),
                 "rows_per_expert_max": int(cnt.max()) // nmb, "rows_per_expert_min": int(cnt.min()) // nmb}
        log(f"zipf routing: top-12 gate-mass share {share:.3f}, selected {sel_share:.3f}, "
            f"rows/expert per micro-batch {int(cnt.min()) // nmb}..{int(cnt.max()) // nmb}")
    log(f"slots routed to the selected experts per micro-batch: S={S} (S/T={S / T:.3f})")
    timing = time_step(step, args.steps, args.warmup, not args.eager)
    bd = breakdown_of(step, max(3, min(20, args.steps)))
    log("per-launch ms:", json.dumps(bd))
    c = dict(cfg, fused_shared=True, n_sel_used=0 if fwd_only else cfg["n_sel"])
    if fwd_only:
        c["r"] = 0
    roof = roofline(bd, c, S, pmc=mode == "c3")
    cpu = None
    if mode in ("c3", "c2") and not args.no_cpu_baseline:
        log("timing the CPU baseline (the oracle: 1 warmup + median of 5 full passes) ...")
        cpu = cpu_baseline(x, W, ex, lora, gy, cfg, fwd_only)
    emit(METRIC if mode == "c3" else QWEN_METRICS[mode], T * nmb, args, timing, QWEN_NAMES[mode],
         {"selected_slots": S, "micro_batches": nmb}, roof, bd, cpu, **extra)


F32_MFMA_PEAK = 157.3e12    # FLOP/s, MI355X dense fp32 MFMA


def run_c3f32(args, dev):
    """c3f32: the C3 layer (same shapes, routing, selected experts and LoRA) with float32 activations and float32
    floating weights, the int4 bank of dtype fp32 (the reference's fp32 models: Int4Experts.from_bf16 of fp32
    weights), fwd+bwd on the fp32 kernels of include/smel_f32.h; eager launches. Roofline of the longest routed-expert
    GEMM against the dense fp32 MFMA peak."""
    from smel.moe import Int4Experts, LayerExperts, moe_forward
    cfg = dict(QWEN)
    log("building the c3 layer in fp32 (int4 quantization on the GPU) ...")
    x, W, ex, lora, gy = build_qwen_layer(dev, cfg)
    W32 = {k: v.float().contiguous() for k, v in W.items()}
    ex32 = LayerExperts(Int4Experts(ex.frozen.gu, ex.frozen.dn, dtype=torch.float32), ex.sel_ids,
                        ex.sel_gate_up.float(), ex.sel_down.float(), group=32, act=cfg["act"])
    xg = x.float().requires_grad_(True)
    gy32 = gy.float()
    params = list(lora.parameters())
    seen = []

    def step(stats=None):
        for p in params:
            p.grad = None
        xg.grad = None
        moe_forward(xg, W32, ex32, cfg["K"], lora, stats=stats).backward(gy32)

    step(stats=lambda p, v, i: seen.append(i))
    sel = torch.zeros(cfg["E"], dtype=torch.bool, device=dev)
    sel[ex.sel_ids.to(dev)] = True
    S = int(sel[seen[0]].sum())
    timing = time_step(step, args.steps, args.warmup, False)
    bd = breakdown_of(step, max(3, min(10, args.steps)))
    log("per-launch ms:", json.dumps(bd))
    T, H, I, K = cfg["T"], cfg["H"], cfg["I"], cfg["K"]
    TK = T * K
    flops = {"gemm_f32_ex_gu": 2 * TK * H * 2 * I, "gemm_f32_ex_dn": 2 * TK * I * H,
             "gemm_f32_ex_dn_bwd": 2 * TK * H * I, "gemm_f32_ex_gu_bwd": 2 * TK * 2 * I * H}
    dom = max(flops, key=lambda k: bd.get(k, 0.0))
    ach = flops[dom] / (bd[dom] * 1e-3)
    roof = {"kernel": dom, "bound": "mfma", "achieved": round(ach / 1e12, 2), "peak": F32_MFMA_PEAK / 1e12,
            "unit": "TFLOP/s", "frac": round(ach / F32_MFMA_PEAK, 4), "traffic": None, "flops_per_launch": flops[dom],
            "avg_launch_ms": bd[dom]}
    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU baseline (the oracle, fp32: 1 warmup + median of 5 full passes) ...")
        cpu = cpu_baseline(x, W, ex, lora, gy, cfg)
    emit("MoE layer fwd+bwd tokens/s with fp32 activations (Qwen3.6 shape, T=4092)", T, args, timing,
         "C3 in fp32: the C3 layer with float32 activations and weights, int4 bank dequantized to fp32, fp32 MFMA",
         {"selected_slots": S}, roof, bd, cpu, dtype="f32")


def run_gemma(args, dev):
    cfg = GEMMA
    log("building the c4 Gemma-4-style block (int4 quantization on the GPU) ...")
    h, a, W, ex, lora, gy = build_gemma_block(dev, cfg)
    hg, ag = (t.clone().requires_grad_(True) for t in (h, a))
    params = list(lora.parameters())
    seen = {}

    def step(stats=None):
        for t in (hg, ag):
            t.grad = None
        for p in params:
            p.grad = None
        gemma_block(hg, ag, W, ex, lora, cfg["K"], stats=stats).backward(gy)

    step(stats=lambda p, v, i: seen.update(topi=i))
    sel = torch.zeros(cfg["E"], dtype=torch.bool, device=dev)
    sel[ex.sel_ids.to(dev)] = True
    S = int(sel[seen["topi"]].sum())
    log(f"slots routed to the selected experts: S={S} (S/T={S / cfg['T']:.3f})")
    timing = time_step(step, args.steps, args.warmup, not args.eager)
    bd = breakdown_of(step, max(3, min(20, args.steps)))
    log("per-launch ms:", json.dumps(bd))
    roof = roofline(bd, dict(cfg, fused_shared=False), S)
    emit("MoE block fwd+bwd tokens/s (Gemma-4-26B-A4B shape, T=4096)", cfg["T"], args, timing,
         "C4: Gemma-4-26B-A4B-style MoE block fwd+bwd from the attention output on: 6 RMSNorms, route_gemma4, 128 "
         "GELU-tanh experts I=704 top-8 (116 int4 g64 + 12 bf16 LoRA r16), dense GeGLU MLP 2112 + LoRA r16, residual "
         "adds and layer scalar, T=4096, H=2816",
         {"selected_slots": S}, roof, bd, None)


def _cpu_threads():
    """Threads for the CPU baseline: every CPU this process may run on, capped at the job's CPU share when the
    environment states one (OMP_NUM_THREADS on the GPU boxes), since more threads than that share oversubscribe."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    share = os.environ.get("OMP_NUM_THREADS", "")
    return min(n, int(share)) if share.isdigit() and int(share) > 0 else n


def _physical_cores():
    """Distinct (physical id, core id) pairs of /proc/cpuinfo, or None."""
    try:
        cores, phys = set(), "0"
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("physical id"):
                phys = ln.split(":", 1)[1].strip()
            elif ln.startswith("core id"):
                cores.add((phys, ln.split(":", 1)[1].strip()))
        return len(cores) or None
    except OSError:
        return None


def cpu_baseline(x, W, ex, lora, gy, cfg, fwd_only=False):
    """The oracle (CPU restatement of the reference's CPU torch path, fp32) on the same layer: 1 warmup pass, then
    the median of 5 timed passes (forward only for C2, forward with autograd + backward for C3)."""
    from oracle import moe_ref as R
    threads = _cpu_threads()
    torch.set_num_threads(threads)
    ol = R.OracleLayer.from_api(W, ex, lora)
    ol.deq_dtype = torch.bfloat16
    assert ol.shared is not None and ol.shared["down"].shape[1] == cfg["Is"]
    xc, gc = x.detach().cpu(), gy.detach().cpu()

    def one():
        if fwd_only:
            with torch.no_grad():
                R.moe_forward(xc, ol, cfg["K"], dtype=torch.float32)
        else:
            R.moe_forward_backward(xc, ol, cfg["K"], gc, dtype=torch.float32)

    one()
    ts = []
    for _ in range(5):
        t0 = time.perf_counter()
        one()
        ts.append(time.perf_counter() - t0)
    dt = statistics.median(ts)
    what = "forward" if fwd_only else "fwd+bwd"
    return {"value": round(cfg["T"] / dt, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{what} of the full layer (T={cfg['T']}) by the oracle, fp32: 1 warmup + median of 5 passes "
                      f"= {dt:.2f} s (range {min(ts):.2f}-{max(ts):.2f}); torch threads={threads}; host: "
                      f"{os.cpu_count()} logical CPUs, {_physical_cores()} physical cores, {_cpu_model()}"}


COPY_BYTES = 1 << 30


def copy_calibration():
    """A device-to-device copy of exactly COPY_BYTES bytes (read COPY_BYTES, write COPY_BYTES), 5 launches."""
    src = torch.randint(0, 255, (COPY_BYTES,), dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy calibration: 5 copies of {COPY_BYTES} bytes")


def run_peaks(args, dev):
    """The achievable peaks of this GPU, by kernels that do nothing else (include/smel_probe.h): the MFMA-only loop
    (v_mfma_f32_32x32x16_bf16, eight independent accumulators per wave, 2 workgroups of 4 waves per CU), a streaming
    read and a device copy of 2 GiB (16 bytes per lane, grid-stride, over a sweep of grid sizes: the best is kept),
    and the platform library's bf16 GEMM (torch.mm on hipBLASLt, 8192^3) for comparison. HIP events on the launching
    stream, best of 5 launches after one warmup."""
    from smel import _lib as L
    cus = torch.cuda.get_device_properties(dev).multi_processor_count

    def best_ms(fn, reps=5):
        fn()
        ts = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            b.synchronize()
            ts.append(a.elapsed_time(b))
        return min(ts)

    blocks, iters = 2 * cus, 4000
    out = torch.empty(blocks * 256, dtype=torch.float32, device=dev)
    ms = best_ms(lambda: L.call("smel_probe_mfma", L.ptr(out), blocks, iters, L.stream()))
    mfma = blocks * 4 * iters * 8 * 32768 / (ms * 1e-3)
    log(f"MFMA loop: {mfma / 1e12:.1f} TFLOP/s")
    nbytes = 2 << 30
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    reads, copies = {}, {}
    for grid in (1024, 2048, 4096, 8192):
        sink = torch.empty(grid * 256, dtype=torch.int32, device=dev)
        reads[grid] = nbytes / (best_ms(lambda: L.call("smel_probe_read", L.ptr(src), nbytes, L.ptr(sink), grid,
                                                       L.stream())) * 1e-3)
        copies[grid] = 2 * nbytes / (best_ms(lambda: L.call("smel_probe_copy", L.ptr(src), L.ptr(dst), nbytes, grid,
                                                            L.stream())) * 1e-3)
    del src, dst
    n = 8192
    a = torch.randn(n, n, device=dev).to(torch.bfloat16)
    b = torch.randn(n, n, device=dev).to(torch.bfloat16)
    c = torch.empty(n, n, device=dev, dtype=torch.bfloat16)
    gemm = 2 * n ** 3 / (best_ms(lambda: torch.mm(a, b, out=c)) * 1e-3)
    rg, cg = max(reads, key=reads.get), max(copies, key=copies.get)
    res = {"mfma_loop_tflops": round(mfma / 1e12, 1), "hipblaslt_bf16_gemm_8192_tflops": round(gemm / 1e12, 1),
           "read_gbps": round(reads[rg] / 1e9), "read_grid": rg, "copy_gbps": round(copies[cg] / 1e9), "copy_grid": cg,
           "read_gbps_by_grid": {k: round(v / 1e9) for k, v in reads.items()},
           "copy_gbps_by_grid": {k: round(v / 1e9) for k, v in copies.items()}, "compute_units": cus}
    print(json.dumps({"metric": "achievable peaks of this GPU (MFMA-only loop, streaming read, device copy)",
                      "value": res["mfma_loop_tflops"], "unit": "TFLOP/s", "n_gpus": 1, "steps": 5, "warmup": 1,
                      "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                      "dtype": "bf16", "data": "synthetic", "config": {"workload": "peaks", "copy_bytes": nbytes},
                      "published": {"mfma_bf16_tflops": MFMA_BF16_PEAK / 1e12, "hbm_gbps": HBM_PEAK / 1e9},
                      "measured": res}), flush=True)


def _cpu_model():
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


NORM_SHAPES = dict(T=4092, H=2048, NQ=16, NKV=2, HD=256, NV=32, VD=128)


def run_norms(args, dev):
    """One step = forward and backward of every RMSNorm of a Qwen3.6 block (smel/layer_runner.py:174-175, 212,
    285-290 call them): C-ABI launches on preallocated buffers, each tagged for the per-kernel breakdown."""
    from smel import _lib
    c = NORM_SHAPES
    T, H, HD, VD = c["T"], c["H"], c["HD"], c["VD"]
    g = torch.Generator(device=dev).manual_seed(0)
    rn = lambda *sh, s=1.0: (torch.randn(*sh, generator=g, device=dev) * s).to(torch.bfloat16)
    P = _lib.ptr
    bufs = {"h": rn(T, H), "a": rn(T, H), "qg": rn(T, c["NQ"], 2 * HD), "k": rn(T, c["NKV"], HD),
            "o": rn(T * c["NV"], VD), "z": rn(T * c["NV"], VD)}
    w = {"in": rn(H, s=0.1), "post": rn(H, s=0.1), "q": rn(HD, s=0.1), "k": rn(HD, s=0.1),
         "g": (1 + 0.1 * torch.randn(VD, generator=g, device=dev)).to(torch.bfloat16)}
    # (tag, rows, cols, row stride, input, weight) of the plain norms; outputs and gradients preallocated
    plain = [("in_norm", T, H, H, bufs["h"], w["in"]), ("q_norm", T * c["NQ"], HD, 2 * HD, bufs["qg"], w["q"]),
             ("k_norm", T * c["NKV"], HD, HD, bufs["k"], w["k"])]
    out = {tag: (torch.empty(R, C, device=dev, dtype=torch.bfloat16), torch.empty(R, device=dev),
                 rn(R, C), torch.empty(R, C, device=dev, dtype=torch.bfloat16)) for tag, R, C, _, _, _ in plain}
    s_, y_, dx_ = (torch.empty(T, H, device=dev, dtype=torch.bfloat16) for _ in range(3))
    r_add = torch.empty(T, device=dev)
    dy_add, ds_add = rn(T, H), rn(T, H)
    Rg = T * c["NV"]
    yg, dxg, dzg = (torch.empty(Rg, VD, device=dev, dtype=torch.bfloat16) for _ in range(3))
    r_g, do_g = torch.empty(Rg, device=dev), rn(Rg, VD)
    EPS = 1e-6

    def step():
        st = _lib.stream()   # the current stream: a side stream while the step is captured
        for tag, R, C, ld, x, wt in plain:
            y, r, dy, dx = out[tag]
            _lib.call("smel_rmsnorm_fwd", P(x), R, C, ld, P(wt), 2, EPS, 0, P(y), P(r), st, tag=tag + "_fwd")
        _lib.call("smel_add_rmsnorm_fwd", P(bufs["h"]), P(bufs["a"]), T, H, P(w["post"]), 2, EPS, 0, P(s_), P(y_),
                  P(r_add), st, tag="add_norm_fwd")
        _lib.call("smel_gated_rmsnorm_fwd", P(bufs["o"]), P(bufs["z"]), Rg, VD, P(w["g"]), EPS, 0, P(yg), P(r_g),
                  st, tag="gated_norm_fwd")
        _lib.call("smel_gated_rmsnorm_bwd", P(do_g), P(bufs["o"]), P(bufs["z"]), Rg, VD, P(w["g"]), P(r_g), 0,
                  P(dxg), P(dzg), st, tag="gated_norm_bwd")
        _lib.call("smel_rmsnorm_bwd", P(dy_add), P(s_), T, H, H, P(w["post"]), 2, P(r_add), P(ds_add), 0, P(dx_),
                  st, tag="add_norm_bwd")
        for tag, R, C, ld, x, wt in plain:
            y, r, dy, dx = out[tag]
            _lib.call("smel_rmsnorm_bwd", P(dy), P(x), R, C, ld, P(wt), 2, P(r), None, 0, P(dx), st,
                      tag=tag + "_bwd")

    # algorithmic HBM bytes per launch: every operand read once, every result written once (bf16 rows, bf16
    # weight, fp32 rstd)
    nbytes = {}
    for tag, R, C, _, _, _ in plain:
        nbytes[tag + "_fwd"] = 2 * R * C * 2 + C * 2 + R * 4
        nbytes[tag + "_bwd"] = 3 * R * C * 2 + C * 2 + R * 4
    nbytes["add_norm_fwd"] = 4 * T * H * 2 + H * 2 + T * 4
    nbytes["add_norm_bwd"] = 4 * T * H * 2 + H * 2 + T * 4
    nbytes["gated_norm_fwd"] = 3 * Rg * VD * 2 + VD * 2 + Rg * 4
    nbytes["gated_norm_bwd"] = 5 * Rg * VD * 2 + VD * 2 + Rg * 4
    timing = time_step(step, args.steps, args.warmup, graph=not args.eager)
    bd = breakdown_of(step, 20)
    dom = max(bd, key=bd.get)
    B, t = nbytes[dom], bd[dom] * 1e-3
    roof = {"kernel": dom, "bound": "hbm", "achieved": round(B / t / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
            "frac": round(B / t / HBM_PEAK, 4), "traffic": measured_traffic(dom), "bytes_per_launch": B,
            "avg_launch_ms": bd[dom],
            "step_bytes": sum(nbytes.values()),
            "step_frac": round(sum(nbytes.values()) / (timing[1] * 1e-3) / HBM_PEAK, 4)}
    cpu = None
    if not args.no_cpu_baseline:
        cpu = norms_cpu_baseline(bufs, w, plain, dict(dy=out, dy_add=dy_add, ds_add=ds_add, do_g=do_g), c)
    emit("RMSNorm family fwd+bwd tokens/s (Qwen3.6 block norms, T=4092)", T, args, timing, "norms",
         {"shapes": "in/post norm [T,2048], q norm [T,16,256] of [T,16,512], k norm [T,2,256], gated [T*32,128]"},
         roof, bd, cpu)


def norms_cpu_baseline(bufs, w, plain, grads, c):
    """The oracle's numpy restatement of the reference's norm kernels (fp32, one thread) on the same step."""
    from oracle import norm_ref as N
    f = lambda t: t.detach().float().cpu().numpy()
    T, H, HD, VD = c["T"], c["H"], c["HD"], c["VD"]
    xs = {"in_norm": f(bufs["h"]), "q_norm": f(bufs["qg"])[..., :HD].reshape(-1, HD),
          "k_norm": f(bufs["k"]).reshape(-1, HD)}
    ins = {"post": f(w["post"]), "g": f(w["g"])}
    dys = {tag: f(grads["dy"][tag][2]) for tag in xs}
    a, o, z, dyo = f(bufs["a"]), f(bufs["o"]), f(bufs["z"]), f(grads["do_g"])
    dy_add, ds_add = f(grads["dy_add"]), f(grads["ds_add"])
    t0 = time.perf_counter()
    for tag, _, _, _, _, wt in plain:
        _, r = N.rmsnorm_fwd(xs[tag], f(wt), 1e-6, 2)
        N.rmsnorm_bwd(dys[tag], xs[tag], f(wt), 2, r)
    s, _, r = N.add_rmsnorm_fwd(xs["in_norm"], a, ins["post"], 1e-6, 2)
    N.rmsnorm_bwd(dy_add, s, ins["post"], 2, r, ds_add)
    _, r = N.gated_fwd(o, z, ins["g"], 1e-6)
    N.gated_bwd(dyo, o, z, ins["g"], r)
    dt = time.perf_counter() - t0
    return {"value": round(T / dt, 1), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"1 fwd+bwd pass of the same norms (T={T}), numpy fp32, {dt:.2f} s, cpu={_cpu_model()}"}


PCIE_GEN5_X16 = 64e9   # B/s per direction, the host link's nominal peak


def run_stream(args, dev):
    """Layer-major streaming of the C3 layer (smel/stream.py:39-114 in the reference; bench_layer.py:119-127 times
    the bank's host -> device copy from pinned memory)."""
    from smel import stream
    from smel.moe import moe_forward
    cfg = dict(QWEN)
    log("building the C3 layer ...")
    x, W, ex, lora, gy = build_qwen_layer(dev, cfg)
    t = {f"experts.gate_up.{k}": v for k, v in ex.frozen.gu.items()}
    t.update({f"experts.down.{k}": v for k, v in ex.frozen.dn.items()})
    t.update({"experts.sel.ids": ex.sel_ids.cpu(), "experts.sel.gate_up": ex.sel_gate_up,
              "experts.sel.down": ex.sel_down})
    t.update({k: v for k, v in W.items() if not k.endswith("gate_up_proj.weight")})
    t = {k: v.detach().cpu() for k, v in t.items()}
    NL = 4
    xg = x.clone().requires_grad_(True)
    params = list(lora.parameters())

    def layer_step(LW):
        for p in params:
            p.grad = None
        xg.grad = None
        moe_forward(xg, LW.W, LW.experts, cfg["K"], lora).backward(gy)

    res = {}
    for ns in (1, 2):
        stream.N_COPY_STREAMS = ns
        src = stream.PinnedSource({0: t}, max_on_gpu=2)
        P = src.pinned[0]
        src.pinned = {l: P for l in range(NL)}
        src.get(0)                                  # first upload: the one host sync (fast-dequant check)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 6
        e0.record()
        for i in range(1, reps + 1):
            src.get(i % NL)
        e1.record()
        torch.cuda.synchronize()
        ms_stage = e0.elapsed_time(e1) / reps
        res[ns] = ms_stage
        log(f"{ns} copy stream(s): stage (copy + pack) {ms_stage:.2f} ms per layer, {P.nbytes / 1e6:.1f} MB, "
            f"{P.nbytes / ms_stage / 1e6:.1f} GB/s")
        src.close()
    ns = 2 if res[2] <= res[1] else 1
    stream.N_COPY_STREAMS = ns
    src = stream.PinnedSource({0: t}, max_on_gpu=2)
    P = src.pinned[0]
    src.pinned = {l: P for l in range(NL)}
    LW = src.get(0)
    layer_step(LW)
    torch.cuda.synchronize()
    # copy-only rate: the same bytes without packing, pinned -> the slot arena
    import ctypes
    from smel import _lib
    slot = src.slots[0]
    evs = [stream._Event() for _ in range(ns)]
    streams = (ctypes.c_void_p * ns)(*[c.cuda_stream for c in src.copy[:ns]])
    done = (ctypes.c_void_p * ns)(*[e.h for e in evs])
    reg = (_lib.H2DRegion * 1)(_lib.H2DRegion(slot.arena.data_ptr(), P.host.data_ptr(), P.nbytes))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(5):
        _lib.call("smel_h2d_regions", reg, 1, stream.CHUNK_BYTES, streams, done, ns, None)
    torch.cuda.synchronize()
    ms_copy = (time.perf_counter() - t0) / 5 * 1e3
    torch.autograd.graph.increment_version(slot.arena)
    src.close()
    src = stream.PinnedSource({0: t}, max_on_gpu=2)
    src.pinned = {l: P for l in range(NL)}
    P.fast = dict(P.fast)

    def step():
        for l in range(NL):
            LW = src.get(l)
            src.prefetch((l + 1) % NL)
            layer_step(LW)

    torch.cuda.synchronize()
    for _ in range(max(1, args.warmup // 5)):
        step()
    torch.cuda.synchronize()
    n = max(1, args.steps // 10)
    t0 = time.perf_counter()
    for _ in range(n):
        step()
    torch.cuda.synchronize()
    ms_layer = (time.perf_counter() - t0) / n / NL * 1e3
    resident = time_step(lambda: layer_step(LW), 10, 3, graph=False)[1]
    log(f"streamed layer {ms_layer:.2f} ms, resident (eager) {resident:.3f} ms, copy {ms_copy:.2f} ms")
    rate = P.nbytes / (ms_copy * 1e-3)
    roof = {"kernel": "h2d_copy", "bound": "pcie", "achieved": round(rate / 1e9, 1), "peak": PCIE_GEN5_X16 / 1e9,
            "unit": "GB/s", "frac": round(rate / PCIE_GEN5_X16, 4), "traffic": None, "bytes_per_launch": P.nbytes,
            "avg_launch_ms": round(ms_copy, 3)}
    emit("streamed MoE layer fwd+bwd tokens/s (C3, weights staged from pinned host memory per layer)", cfg["T"],
         args, ("eager_layer_major", ms_layer, ms_layer), "stream",
         {"layer_bytes": P.nbytes, "layer_ids": NL, "copy_streams": ns, "chunk_bytes": stream.CHUNK_BYTES},
         roof, {"stage_ms_1_stream": round(res[1], 3), "stage_ms_2_streams": round(res[2], 3),
                "copy_ms": round(ms_copy, 3), "resident_layer_ms": round(resident, 3)}, None)


def run_quant(args, dev):
    """quantize_int4 (smel/quant.py:14-44) of a whole C2-shaped bank on the GPU: HIP kernel time per bank, and the
    oracle's restatement of the same algorithm as torch ops on the host CPU (sampled) as the baseline."""
    from smel import quant
    c = QWEN
    E, H, I = c["E"], c["H"], c["I"]
    g = torch.Generator(device=dev).manual_seed(0)
    gu = (torch.randn(E, 2 * I, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    dn = (torch.randn(E, H, I, generator=g, device=dev) * 0.02).to(torch.bfloat16)

    def step():
        quant.quantize_int4(gu, 64)
        quant.quantize_int4(dn, 64)

    timing = time_step(step, max(3, args.steps // 10), 2, graph=False)
    bd = breakdown_of(step, 3)
    ms = timing[1]
    nbytes = (gu.numel() + dn.numel()) * 2 + (gu.numel() + dn.numel()) // 2 + (gu.numel() + dn.numel()) // 64 * 4
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import moe_ref as R
        w = gu[:1].cpu()
        torch.set_num_threads(_cpu_threads())
        t0 = time.perf_counter()
        R.quantize_int4(w, 64)
        dt = time.perf_counter() - t0
        per_bank_s = dt * E * 1.5
        cpu = {"value": round(1 / per_bank_s, 4), "unit": "banks/s", "cores": torch.get_num_threads(),
               "kind": "port", "sample": f"1 expert's gate_up ({2 * I}x{H}) by the oracle (torch ops) on the CPU in "
                                         f"{dt:.2f} s, scaled to the bank (x{E * 1.5:.0f}), cpu={_cpu_model()}"}
    t = bd.get("smel_quantize_int4", ms / 2)
    roof = {"kernel": "quantize_int4_reg_kernel<64>", "bound": "hbm", "achieved": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": round(nbytes / (ms * 1e-3) / HBM_PEAK, 4),
            "traffic": None, "bytes_per_launch": nbytes // 2, "avg_launch_ms": t,
            "note": "VALU-bound: 5 candidates x (2 divisions + 10 operations) per weight"}
    out_ms = {"hip_bank_ms": round(ms, 3)}
    log(f"bank quantized in {ms:.2f} ms")
    print(json.dumps({"metric": "int4 bank quantization banks/s (C2 bank: 256 experts, group 64, 5 clip factors)",
                      "value": round(1e3 / ms, 2), "unit": "banks/s", "n_gpus": 1, "steps": timing and args.steps,
                      "warmup": 2, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
                      "vs_baseline": None, "dtype": "f32", "data": "synthetic bf16 weights ~N(0, 0.02)",
                      "config": {"workload": "quant", "experts": E, "gate_up": [2 * I, H], "down": [H, I],
                                 "group": 64}, "roofline": roof, "breakdown_ms": {**bd, **out_ms},
                      "cpu_baseline": cpu}), flush=True)


# token_chunk 4096: one pass over the vocabulary for the whole sequence (the results are those of any chunking)
CE_SHAPE = dict(T=4092, H=2048, V=248320, token_chunk=4096, vocab_chunk=32768)


def run_ce(args, dev):
    """chunked_ce (smel/loss.py:149-156) loss and gradient for one sequence of the Qwen3.6 shape: per vocabulary
    chunk the logits GEMM with the online softmax in its epilogue (smel_ce_logits), the statistics fold
    (smel_ce_stats) and the gradient GEMM p W (smel_ce_grad), both GEMMs on MFMA; the roofline line is the whole
    step's MFMA rate, with each GEMM's own rate per launch beside it."""
    from smel import loss as LS
    c = CE_SHAPE
    T, H, V = c["T"], c["H"], c["V"]
    g = torch.Generator(device=dev).manual_seed(0)
    h = torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16).requires_grad_(True)
    W = (torch.randn(V, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    tgt = torch.randint(0, V, (T,), generator=g, device=dev)
    head = LS.LMHead(weight=W, vocab_chunk=c["vocab_chunk"])

    def step():
        h.grad = None
        LS.chunked_ce(h, head, tgt, denom=float(T), token_chunk=c["token_chunk"]).backward()

    timing = time_step(step, max(3, args.steps // 10), 2, graph=False)
    bd = breakdown_of(step, 2)
    ms = timing[1]
    flops = 4 * T * V * H                         # logits GEMM + gradient GEMM, 2 T V H each
    chunks, _ = head._kernel_chunks()
    per_launch = 2 * T * V * H / len(chunks)      # one GEMM of one vocabulary chunk, averaged over the chunks
    per_kernel = {k: round(per_launch / (bd[k] * 1e-3) / 1e12, 1) for k in ("smel_ce_logits", "smel_ce_grad")
                  if k in bd}
    roof = {"kernel": "whole step (smel_ce_logits + smel_ce_grad on MFMA, smel_ce_stats / _finish)", "bound": "mfma",
            "achieved": round(flops / (ms * 1e-3) / 1e12, 1), "peak": MFMA_BF16_PEAK / 1e12, "unit": "TFLOP/s",
            "frac": round(flops / (ms * 1e-3) / MFMA_BF16_PEAK, 4), "traffic": None, "flops_per_step": flops,
            "per_launch_tflops": per_kernel}
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import loss_ref as LR
        torch.set_num_threads(_cpu_threads())
        ns = 32
        t0 = time.perf_counter()
        LR.full_ce(h[:ns].float(), W.float(), tgt[:ns], 0.0, float(T))
        dt = time.perf_counter() - t0
        cpu = {"value": round(ns / dt, 1), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"{ns} tokens through the full-logit fp64 oracle (loss + gradient) in {dt:.2f} s, "
                         f"cpu={_cpu_model()}"}
    emit("chunked CE loss+grad tokens/s (Qwen3.6 head: hidden 2048, vocabulary 248320)", T, args, timing, "ce",
         dict(c), roof, bd, cpu)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", choices=("c3", "c2", "c4", "c5", "c3f32", "norms", "stream", "quant", "ce", "peaks"),
                    default="c3")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true", help="time eager launches only (no HIP graph replay)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device copy of COPY_BYTES bytes 5 times (the reference point that scales "
                         "the FETCH_SIZE / WRITE_SIZE counters of a rocprofv3 --pmc run to bytes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the MoE hot path here runs on one MI355X and has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    from smel import _lib
    _lib.load()
    dev = torch.device("cuda:0")
    if args.workload == "c4":
        run_gemma(args, dev)
    elif args.workload == "norms":
        run_norms(args, dev)
    elif args.workload == "stream":
        run_stream(args, dev)
    elif args.workload == "quant":
        run_quant(args, dev)
    elif args.workload == "ce":
        run_ce(args, dev)
    elif args.workload == "peaks":
        run_peaks(args, dev)
    elif args.workload == "c3f32":
        run_c3f32(args, dev)
    else:
        run_qwen(args, dev, args.workload)


if __name__ == "__main__":
    main()
