"""The packed-layer format and the LoRA merge of smel.pack on the CPU, against the reference's own outputs
(tests/golden/pack_layer.safetensors, written by the reference's pack_layer / merge_experts / merge_mlp,
smel/pack.py:8-45) and against the merge's formula in fp64.

The int4 banks need the GPU (smel_quantize_int4) and are compared in test_gpu_pack.py; here the golden banks pin the
oracle's quantizer at 20 experts (the 16-expert slices), and every other part of the format is compared bit for bit:
names and their order, dtypes (bf16 for floating tensors, A_log / dt_bias and integer tensors kept), values."""
import json
import os

import pytest
import torch
from safetensors import safe_open
from safetensors.torch import load_file

from oracle import moe_ref as R
from smel import pack
from smel.lora import ExpertsLoRA, MLPLoRA

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "pack_layer.safetensors")
SEL = [3, 17]
LORA = ("A_gate", "A_up", "A_down", "B_gate", "B_up", "B_down")


@pytest.fixture(scope="module")
def gold():
    with safe_open(GOLDEN, "pt") as f:
        order = json.loads(f.metadata()["order"])
    return load_file(GOLDEN), order


def _inputs(g, order=None):
    """The layer dict; with ``order``, its dense tensors in the order the reference received them (the file itself
    stores names sorted), so the output order can be compared."""
    t = {k[3:]: v for k, v in g.items() if k.startswith("in.")}
    if order is None:
        return t
    dense = [k for k in order["nosel"] if not k.startswith("experts.")]
    return {**{k: t[k] for k in dense}, **{k: v for k, v in t.items() if k not in dense}}


def _bits(t):
    return t.view(torch.int16) if t.dtype in (torch.bfloat16, torch.float16) else t


@pytest.mark.parametrize("tag,ids", [("sel", SEL), ("nosel", None)])
def test_dense_and_selected_parts(gold, tag, ids):
    g, order = gold
    t = _inputs(g, order)
    got = pack._dense_part(t, torch.bfloat16)
    got.update(pack._selected_part(t, ids, torch.bfloat16))
    want = [k for k in order[tag] if not k.startswith(("experts.gate_up.", "experts.down."))]
    assert list(got) == want
    for k in want:
        ref = g[f"{tag}.{k}"]
        assert got[k].dtype == ref.dtype and got[k].shape == ref.shape, k
        assert torch.equal(_bits(got[k]), _bits(ref)), k
        assert got[k].is_contiguous()
    kept = {"linear_attn.A_log", "linear_attn.dt_bias", "conv1d.position_ids"}
    assert {k for k in want if got[k].dtype != torch.bfloat16} == kept | ({"experts.sel.ids"} if ids else set())


def test_golden_banks_pin_the_oracle_quantizer(gold):
    g, _ = gold
    t = _inputs(g)
    for tag, group in (("sel", 64), ("nosel", 32)):
        for name, key in (("gate_up", "mlp.experts.gate_up_proj"), ("down", "mlp.experts.down_proj")):
            pk = R.quantize_int4(t[key], group)
            for field in ("q", "scale", "zero"):
                assert torch.equal(_bits(pk[field]), _bits(g[f"{tag}.experts.{name}.{field}"])), (tag, name, field)


def _loras(g):
    ex = ExpertsLoRA(SEL, 64, 64, r=4, alpha=6.0)
    sh = MLPLoRA(64, 96, r=4, alpha=6.0)
    with torch.no_grad():
        for n in LORA:
            getattr(ex, n).copy_(g["lora.ex_" + n])
            getattr(sh, n).copy_(g["lora.sh_" + n])
    return ex, sh


def test_merge_matches_reference_bits(gold):
    g, _ = gold
    t = _inputs(g)
    ex, sh = _loras(g)
    gu0, dn0 = t["mlp.experts.gate_up_proj"], t["mlp.experts.down_proj"]
    gu, dn = pack.merge_experts(gu0, dn0, ex)
    assert gu.dtype == torch.bfloat16 and gu.data_ptr() != gu0.data_ptr()
    assert torch.equal(_bits(gu[SEL]), _bits(g["merge.gate_up_sel"]))
    assert torch.equal(_bits(dn[SEL]), _bits(g["merge.down_sel"]))
    rest = [e for e in range(gu0.shape[0]) if e not in SEL]
    assert torch.equal(gu[rest], gu0[rest]) and torch.equal(dn[rest], dn0[rest])
    p = "mlp.shared_expert."
    merged = pack.merge_mlp(t[p + "gate_proj.weight"], t[p + "up_proj.weight"], t[p + "down_proj.weight"], sh)
    for n, w in zip(("gate", "up", "down"), merged):
        assert torch.equal(_bits(w), _bits(g["merge.sh_" + n])), n


def test_merge_is_base_plus_scaled_product(gold):
    """Independent of the golden: every merged weight is the bf16 rounding of w + scale B A (fp64), i.e. within half
    a bf16 ulp of it plus the fp32 error of the product; the unmerged weights differ from it by the whole delta."""
    g, _ = gold
    t = _inputs(g)
    ex, sh = _loras(g)
    gu, dn = pack.merge_experts(t["mlp.experts.gate_up_proj"], t["mlp.experts.down_proj"], ex)
    I = 64
    for j, e in enumerate(SEL):
        for w_new, w_old, B, A in ((gu[e, :I], t["mlp.experts.gate_up_proj"][e, :I], ex.B_gate[j], ex.A_gate[j]),
                                   (gu[e, I:], t["mlp.experts.gate_up_proj"][e, I:], ex.B_up[j], ex.A_up[j]),
                                   (dn[e], t["mlp.experts.down_proj"][e], ex.B_down[j], ex.A_down[j])):
            exact = w_old.double() + 1.5 * B.detach().double() @ A.detach().double()
            ulp = torch.finfo(torch.bfloat16).eps * exact.abs()
            assert torch.all((w_new.double() - exact).abs() <= 0.5 * ulp + 1e-7)
            assert (w_old.double() - exact).abs().max() > 1e-3


def test_pack_layer_errors():
    t = {"mlp.gate.weight": torch.zeros(4, 64), "mlp.experts.gate_up_proj": torch.zeros(4, 8, 64)}
    with pytest.raises(KeyError):
        pack.pack_layer(t, [1])
    t["mlp.experts.down_proj"] = torch.zeros(4, 64, 48)
    with pytest.raises(AssertionError):          # down's input dim 48 is not a multiple of the group
        pack.pack_layer(t, None, 64)
