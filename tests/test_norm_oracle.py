"""Pins the CPU restatement of the RMSNorm kernels (oracle/norm_ref.py) against what does not share its formulas:
fp64 closed forms, fp64 autograd of the textbook forward (so a dropped term or a wrong sign in the backward formula
fails), torch's own 16-bit add, and the reference's torch code (smel/layer_runner.py:110-138) at the reference
test's tolerances (tests/test_norm.py:35-98). Also the host-side argument checks of the C-ABI norm entry points
(no kernel runs: every case is rejected before a launch). CPU only."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import norm_ref as N

EPS = 1e-6
SHAPES = [(37, 2048), (3, 29, 2816), (64, 16, 256), (50, 2, 256), (40, 100)]   # tests/test_norm.py:35
TDT = {"bf16": torch.bfloat16, "fp16": torch.float16}
ULP_REL = {"bf16": 2.0 ** -8, "fp16": 2.0 ** -11}   # half an ulp, relative
ULP_ABS = {"bf16": 2.0 ** -134, "fp16": 2.0 ** -25}  # half an ulp of the subnormals


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def inputs(shape, dt, seed, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(shape, generator=g) * scale).to(TDT[dt]).float()
    w = (torch.randn(shape[-1], generator=g) * 0.1).to(TDT[dt]).float()
    dy = (torch.randn(shape, generator=g) + 0.5 * x).to(TDT[dt]).float()   # correlated with x: mean(g xhat) is large
    return x.numpy(), w.numpy(), dy.numpy()


def closed_fwd64(x, w, eps, w_mode):
    x = torch.as_tensor(x, dtype=torch.float64)
    wp = {0: torch.ones(x.shape[-1], dtype=torch.float64), 1: torch.as_tensor(w, dtype=torch.float64),
          2: 1 + torch.as_tensor(w, dtype=torch.float64)}[w_mode]
    return x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps) * wp


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("w_mode", [0, 1, 2])
@pytest.mark.parametrize("shape", SHAPES)
def test_rmsnorm_fwd_closed_form(shape, w_mode, dt):
    x, w, _ = inputs(shape, dt, 0)
    y, r = N.rmsnorm_fwd(x, w, EPS, w_mode, dt)
    y64 = closed_fwd64(x, w, EPS, w_mode).numpy()
    assert np.all(np.abs(y - y64) <= ULP_REL[dt] * 1.001 * np.abs(y64) + ULP_ABS[dt])
    r64 = 1 / np.sqrt((x.astype(np.float64) ** 2).mean(-1) + EPS)
    assert np.max(np.abs(r - r64) / r64) < 1e-6
    # the reference's torch code, at the reference test's bar
    xt = torch.as_tensor(x).to(TDT[dt])
    wt = None if w_mode == 0 else torch.as_tensor(w).to(TDT[dt])
    yt = N.torch_rmsnorm(xt, wt, EPS, plus_one=(w_mode == 2)).float().numpy()
    assert rel(y, yt) < 1e-4


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("with_ds", [False, True])
@pytest.mark.parametrize("w_mode", [0, 1, 2])
@pytest.mark.parametrize("shape", SHAPES)
def test_rmsnorm_bwd_autograd(shape, w_mode, with_ds, dt):
    x, w, dy = inputs(shape, dt, 1)
    ds = inputs(shape, dt, 2)[2] if with_ds else None
    _, r = N.rmsnorm_fwd(x, w, EPS, w_mode, dt)
    dx = N.rmsnorm_bwd(dy, x, w, w_mode, r, ds, dt)
    x64 = torch.as_tensor(x, dtype=torch.float64).requires_grad_(True)
    y64 = closed_fwd64(x64, w, EPS, w_mode)
    (y64 * torch.as_tensor(dy, dtype=torch.float64)).sum().backward()
    ref = x64.grad.numpy() + (ds.astype(np.float64) if with_ds else 0)
    assert rel(dx, ref) < {"bf16": 3e-3, "fp16": 4e-4}[dt]


def test_rmsnorm_bwd_catches_a_dropped_term():
    """The autograd check above is sharp enough to see the mean term of the backward formula."""
    x, w, dy = inputs((37, 2048), "bf16", 1)
    _, r = N.rmsnorm_fwd(x, w, EPS, 2, "bf16")
    x64 = torch.as_tensor(x, dtype=torch.float64).requires_grad_(True)
    (closed_fwd64(x64, w, EPS, 2) * torch.as_tensor(dy, dtype=torch.float64)).sum().backward()
    wrong = N.rnd(r[:, None] * dy * (1 + w), "bf16")   # g only, without - xhat mean(g xhat)
    assert rel(wrong, x64.grad.numpy()) > 3e-2


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("w_mode", [1, 2])
def test_add_rmsnorm(w_mode, dt):
    """tests/test_norm.py:63-86: s equals torch's 16-bit h + x bit for bit; y and the gradient of both inputs
    against fp64."""
    shape = (300, 2048)
    h, w, dy = inputs(shape, dt, 3, scale=1.0)
    x = inputs(shape, dt, 4, scale=1.0)[0]
    ds = inputs(shape, dt, 5)[2]
    s, y, r = N.add_rmsnorm_fwd(h, x, w, EPS, w_mode, dt)
    st = (torch.as_tensor(h).to(TDT[dt]) + torch.as_tensor(x).to(TDT[dt])).float().numpy()
    assert np.array_equal(s, st)
    y64 = closed_fwd64(s, w, EPS, w_mode).numpy()
    assert np.all(np.abs(y - y64) <= ULP_REL[dt] * 1.001 * np.abs(y64) + ULP_ABS[dt])
    d = N.rmsnorm_bwd(dy, s, w, w_mode, r, ds, dt)
    s64 = torch.as_tensor(s, dtype=torch.float64).requires_grad_(True)
    ((s64 * torch.as_tensor(ds, dtype=torch.float64)).sum()
     + (closed_fwd64(s64, w, EPS, w_mode) * torch.as_tensor(dy, dtype=torch.float64)).sum()).backward()
    assert rel(d, s64.grad.numpy()) < {"bf16": 3e-3, "fp16": 4e-4}[dt]


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("shape", [(64 * 32, 128), (37, 2048), (40, 100)])
def test_gated(shape, dt):
    """tests/test_norm.py:89-98 (torch code, 1e-3) and fp64 autograd of y = w x rstd silu(z)."""
    g = torch.Generator().manual_seed(6)
    x = torch.randn(shape, generator=g).to(TDT[dt])
    z = torch.randn(shape, generator=g).to(TDT[dt])
    w = (1 + 0.1 * torch.randn(shape[-1], generator=g)).to(TDT[dt])
    do = torch.randn(shape, generator=g).to(TDT[dt])
    y, r = N.gated_fwd(x.float().numpy(), z.float().numpy(), w.float().numpy(), EPS, dt)
    dx, dz = N.gated_bwd(do.float().numpy(), x.float().numpy(), z.float().numpy(), w.float().numpy(), r, dt)
    xt, zt = x.clone().requires_grad_(True), z.clone().requires_grad_(True)
    yt = N.torch_gated_rmsnorm(xt, zt, w, EPS)
    (yt.float() * do.float()).sum().backward()
    assert rel(y, yt.float().detach().numpy()) < 1e-3
    assert rel(dx, xt.grad.float().numpy()) < 1e-3 and rel(dz, zt.grad.float().numpy()) < 1e-3
    x64 = x.double().requires_grad_(True)
    z64 = z.double().requires_grad_(True)
    y64 = w.double() * x64 / torch.sqrt((x64 * x64).mean(-1, keepdim=True) + EPS) * torch.nn.functional.silu(z64)
    (y64 * do.double()).sum().backward()
    assert rel(y, y64.detach().numpy()) < 1e-2
    assert rel(dx, x64.grad.numpy()) < 2e-2 and rel(dz, z64.grad.numpy()) < 1e-2


# ----------------------------------------------------------------------- host-side checks of the C-ABI entry points


def test_norm_entry_points_reject_bad_arguments():
    from smel import _lib
    L = _lib.load()
    fake = ctypes.c_void_p(1 << 20)   # never dereferenced: every call below fails its checks before a launch
    EINVAL, EUNSUP = -1, -2
    assert L.smel_rmsnorm_fwd(fake, 4, 16385, 16385, None, 0, 1e-6, 0, fake, fake, None) == EUNSUP
    assert L.smel_rmsnorm_fwd(fake, 4, 64, 32, None, 0, 1e-6, 0, fake, fake, None) == EINVAL    # stride < cols
    assert L.smel_rmsnorm_fwd(fake, 4, 64, 64, None, 1, 1e-6, 0, fake, fake, None) == EINVAL    # w_mode 1, no w
    assert L.smel_rmsnorm_fwd(fake, 4, 64, 64, fake, 3, 1e-6, 0, fake, fake, None) == EINVAL    # w_mode 3
    assert L.smel_rmsnorm_fwd(fake, 4, 64, 64, None, 0, 1e-6, 2, fake, fake, None) == EINVAL    # dtype 2
    assert L.smel_rmsnorm_fwd(None, 4, 64, 64, None, 0, 1e-6, 0, fake, fake, None) == EINVAL    # null x
    assert L.smel_rmsnorm_fwd(fake, 0, 64, 64, None, 0, 1e-6, 0, fake, fake, None) == 0         # no rows: no-op
    assert L.smel_rmsnorm_bwd(fake, fake, 4, 0, 0, None, 0, fake, None, 0, fake, None) == EINVAL
    assert L.smel_add_rmsnorm_fwd(fake, None, 4, 64, fake, 2, 1e-6, 0, fake, fake, fake, None) == EINVAL
    assert L.smel_gated_rmsnorm_fwd(fake, fake, 4, 64, None, 1e-6, 0, fake, fake, None) == EINVAL
    assert L.smel_gated_rmsnorm_bwd(fake, fake, fake, -1, 64, fake, fake, 0, fake, fake, None) == EINVAL
    assert b"w_mode" in L.smel_last_error() or len(L.smel_last_error()) > 0
