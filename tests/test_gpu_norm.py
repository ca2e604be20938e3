"""HIP RMSNorm kernels (smel.norm over include/smel_norm.h) against the CPU restatement oracle/norm_ref.py on the
same inputs, through the autograd API: the reference's test shapes and variants (tests/test_norm.py:35-110), both
16-bit dtypes, the strided view, the residual add with and without each gradient, the gated norm, and the edge
cases (no rows, one column, columns not a multiple of 8, an unaligned row start, the 16384-column maximum).

Bar: outputs within one rounding of the oracle's (both compute in fp32 with the same rounding points; only the
order of each row's fp32 sum differs, which can move a value across a rounding boundary), the residual sum bit for
bit, and the reference test's own norm-relative bound (1e-4; 1e-3 for the gated norm); repeated calls bitwise
equal. The gated norm rounds in a chain (forward: round(round(w round(x rstd)) silu(z)); backward:
dn = round(round(dout silu(z)) w) before the row sum), so a last-bit difference of rstd or of exp between the device
and numpy can flip an intermediate rounding and move the result by one ulp of the intermediate: there at most 1 in
10^4 elements may exceed one ulp of their own value, and none one ulp of its row's largest."""
import numpy as np
import pytest
import torch

from oracle import norm_ref as N

pytestmark = pytest.mark.gpu
EPS = 1e-6
TDT = {"bf16": torch.bfloat16, "fp16": torch.float16}
ULP = {"bf16": 2.0 ** -7, "fp16": 2.0 ** -10}   # one ulp, relative
SHAPES = [(37, 2048), (3, 29, 2816), (64, 16, 256), (50, 2, 256), (40, 100)]


@pytest.fixture(scope="module")
def nm():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from smel import norm
    return norm


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def f32(t):
    return t.detach().float().cpu().numpy()


def close(got, want, dt, rel_bar=1e-4, flips=0.0):
    """Within one ulp of the oracle's value, plus a floor of 1e-5 of the row scale for cancelling sums; a fraction
    `flips` of the elements may instead be within one ulp of their row's largest value."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    rowmax = np.abs(want).max(axis=-1, keepdims=True)
    diff = np.abs(got - want)
    bad = diff > ULP[dt] * np.abs(want) + 1e-5 * rowmax + 2.0 ** -24
    assert bad.sum() <= flips * bad.size, f"{bad.sum()} of {bad.size} beyond one ulp; max |diff| {diff.max()}"
    assert not (diff > ULP[dt] * rowmax + 2.0 ** -24).any()
    assert rel(got, want) < rel_bar


def run_rms(nm, x, w, plus_one, dy):
    xg = x.detach().clone().requires_grad_(True)
    y = nm.rmsnorm(xg, w, EPS, plus_one)
    (y.float() * dy.float()).sum().backward()
    return y, xg.grad


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("variant", ["plus_one", "scale", "none"])
@pytest.mark.parametrize("shape", SHAPES)
def test_rmsnorm(nm, shape, variant, dt):
    print(f"rmsnorm {shape} {variant} {dt}", flush=True)
    torch.manual_seed(0)
    x = (torch.randn(shape, device="cuda") * 2).to(TDT[dt])
    w = None if variant == "none" else (torch.randn(shape[-1], device="cuda") * 0.1).to(TDT[dt])
    dy = torch.randn(shape, device="cuda").to(TDT[dt])
    assert nm.supported(x, w)
    w_mode = {"none": 0, "scale": 1, "plus_one": 2}[variant]
    y, dx = run_rms(nm, x, w, variant == "plus_one", dy)
    yo, r = N.rmsnorm_fwd(f32(x), None if w is None else f32(w), EPS, w_mode, dt)
    dxo = N.rmsnorm_bwd(f32(dy), f32(x), None if w is None else f32(w), w_mode, r, None, dt)
    assert y.dtype == x.dtype and y.shape == x.shape and dx.shape == x.shape
    close(f32(y), yo, dt)
    close(f32(dx), dxo, dt)
    y2, dx2 = run_rms(nm, x, w, variant == "plus_one", dy)
    assert torch.equal(y, y2) and torch.equal(dx, dx2)


def test_rmsnorm_of_a_strided_view(nm):
    """tests/test_norm.py:50-60: q of the gated attention is the first half of each row of q_proj's output."""
    torch.manual_seed(1)
    qg = torch.randn(70, 16, 512, device="cuda").to(torch.bfloat16).requires_grad_(True)
    w = (torch.randn(256, device="cuda") * 0.1).to(torch.bfloat16)
    dy = torch.randn(70, 16, 256, device="cuda").to(torch.bfloat16)
    y = nm.rmsnorm(qg.chunk(2, dim=-1)[0], w, EPS, True)
    (y.float() * dy.float()).sum().backward()
    xq = f32(qg)[..., :256]
    yo, r = N.rmsnorm_fwd(xq, f32(w), EPS, 2, "bf16")
    close(f32(y), yo, "bf16")
    close(f32(qg.grad)[..., :256], N.rmsnorm_bwd(f32(dy), xq, f32(w), 2, r, None, "bf16"), "bf16")
    assert qg.grad[..., 256:].abs().max() == 0


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("plus_one", [True, False])
def test_add_rmsnorm(nm, plus_one, dt):
    """tests/test_norm.py:63-86: s bit for bit, both inputs get the same gradient (norm dx + ds, one rounding)."""
    torch.manual_seed(2)
    h = torch.randn(300, 2048, device="cuda").to(TDT[dt])
    x = torch.randn_like(h)
    w = (torch.randn(2048, device="cuda") * 0.1).to(TDT[dt])
    ds, dy = torch.randn_like(h), torch.randn_like(h)
    hg, xg = h.clone().requires_grad_(True), x.clone().requires_grad_(True)
    s, y = nm.add_rmsnorm(hg, xg, w, EPS, plus_one)
    ((s.float() * ds.float()).sum() + (y.float() * dy.float()).sum()).backward()
    w_mode = 2 if plus_one else 1
    so, yo, r = N.add_rmsnorm_fwd(f32(h), f32(x), f32(w), EPS, w_mode, dt)
    assert np.array_equal(f32(s), so)
    close(f32(y), yo, dt)
    do = N.rmsnorm_bwd(f32(dy), so, f32(w), w_mode, r, f32(ds), dt)
    close(f32(hg.grad), do, dt)
    assert torch.equal(hg.grad, xg.grad)


def test_add_rmsnorm_one_output_used(nm):
    """Only y reaches the loss (no ds: the kernel adds nothing), or only s (the norm's backward is skipped)."""
    torch.manual_seed(3)
    h = torch.randn(64, 2048, device="cuda").to(torch.bfloat16)
    x = torch.randn_like(h)
    w = (torch.randn(2048, device="cuda") * 0.1).to(torch.bfloat16)
    dy = torch.randn_like(h)
    hg, xg = h.clone().requires_grad_(True), x.clone().requires_grad_(True)
    s, y = nm.add_rmsnorm(hg, xg, w, EPS, True)
    (y.float() * dy.float()).sum().backward()
    so, _, r = N.add_rmsnorm_fwd(f32(h), f32(x), f32(w), EPS, 2, "bf16")
    close(f32(hg.grad), N.rmsnorm_bwd(f32(dy), so, f32(w), 2, r, None, "bf16"), "bf16")
    hg2 = h.clone().requires_grad_(True)
    s2, _ = nm.add_rmsnorm(hg2, x, w, EPS, True)
    (s2.float() * dy.float()).sum().backward()
    assert torch.equal(hg2.grad, dy)


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("shape", [(64 * 32, 128), (37, 2048), (40, 100), (5, 2816)])
def test_gated_rmsnorm(nm, shape, dt):
    """tests/test_norm.py:89-98."""
    print(f"gated {shape} {dt}", flush=True)
    torch.manual_seed(4)
    x = torch.randn(shape, device="cuda").to(TDT[dt])
    z = torch.randn_like(x)
    w = (1 + 0.1 * torch.randn(shape[-1], device="cuda")).to(TDT[dt])
    do = torch.randn_like(x)
    xg, zg = x.clone().requires_grad_(True), z.clone().requires_grad_(True)
    y = nm.gated_rmsnorm(xg, zg, w, EPS)
    (y.float() * do.float()).sum().backward()
    yo, r = N.gated_fwd(f32(x), f32(z), f32(w), EPS, dt)
    dxo, dzo = N.gated_bwd(f32(do), f32(x), f32(z), f32(w), r, dt)
    close(f32(y), yo, dt, rel_bar=1e-3, flips=1e-4)
    close(f32(xg.grad), dxo, dt, rel_bar=1e-3, flips=1e-4)
    close(f32(zg.grad), dzo, dt, rel_bar=1e-3, flips=1e-4)


@pytest.mark.parametrize("rows,cols", [(0, 2048), (1, 1), (7, 3), (33, 100), (3, 16384), (5, 8200), (300, 2048)])
def test_edge_sizes(nm, rows, cols):
    """No rows, one column, columns not a multiple of 8 (element path), the maximum width, one block per row."""
    print(f"edge {rows}x{cols}", flush=True)
    torch.manual_seed(5)
    x = torch.randn(rows, cols, device="cuda").to(torch.bfloat16)
    w = (torch.randn(cols, device="cuda") * 0.1).to(torch.bfloat16)
    dy = torch.randn_like(x)
    y, dx = run_rms(nm, x, w, True, dy)
    assert y.shape == (rows, cols) and dx.shape == (rows, cols)
    if rows:
        yo, r = N.rmsnorm_fwd(f32(x), f32(w), EPS, 2, "bf16")
        close(f32(y), yo, "bf16")
        close(f32(dx), N.rmsnorm_bwd(f32(dy), f32(x), f32(w), 2, r, None, "bf16"), "bf16")


def test_unaligned_rows(nm):
    """A row start that is not 16-byte aligned takes the element-by-element path; same results."""
    torch.manual_seed(6)
    buf = torch.randn(40 * 256 + 1, device="cuda").to(torch.bfloat16)
    x = buf[1:].view(40, 256)
    w = (torch.randn(256, device="cuda") * 0.1).to(torch.bfloat16)
    dy = torch.randn(40, 256, device="cuda").to(torch.bfloat16)
    y, dx = run_rms(nm, x, w, False, dy)
    ya, dxa = run_rms(nm, x.contiguous(), w, False, dy)
    assert torch.equal(y, ya) and torch.equal(dx, dxa)
    yo, r = N.rmsnorm_fwd(f32(x), f32(w), EPS, 1, "bf16")
    close(f32(y), yo, "bf16")


def test_supported_and_errors(nm):
    """tests/test_norm.py:101-110: fp32 rows, trainable or other-dtype weights and CPU tensors are not the kernels'
    (the caller keeps its torch code for them); the kernels themselves reject a weight of another dtype."""
    x32 = torch.randn(8, 64, device="cuda")
    assert not nm.supported(x32, torch.ones(64, device="cuda"))
    xb = x32.to(torch.bfloat16)
    assert not nm.supported(xb, torch.ones(64, device="cuda", dtype=torch.bfloat16, requires_grad=True))
    assert not nm.supported(xb, torch.ones(64, device="cuda"))
    assert not nm.supported(xb.cpu(), None)
    assert not nm.supported(torch.zeros(2, 16385, device="cuda", dtype=torch.bfloat16), None)
    assert nm.supported(xb, None) and nm.supported(xb, torch.ones(64, device="cuda", dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        nm.rmsnorm(xb, torch.ones(64, device="cuda"), EPS, True)
