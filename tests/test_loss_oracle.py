"""Pins the cross-entropy oracle (oracle/loss_ref.py) on the CPU: its loss against a per-row log-sum-exp written
out in numpy, its softcapped gradient against central finite differences; and the host-side argument checks of
the CE entry points of include/smel_loss.h (no kernel runs)."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import loss_ref as LR


@pytest.mark.parametrize("softcap", [0.0, 30.0])
def test_full_ce_against_numpy(softcap):
    g = torch.Generator().manual_seed(0)
    h, W = torch.randn(9, 16, generator=g), torch.randn(50, 16, generator=g) * 2
    tgt = torch.randint(0, 50, (9,), generator=g)
    loss, _ = LR.full_ce(h, W, tgt, softcap, denom=3.0)
    z = h.double().numpy() @ W.double().numpy().T
    if softcap:
        z = softcap * np.tanh(z / softcap)
    mx = z.max(1, keepdims=True)
    lse = (mx + np.log(np.exp(z - mx).sum(1, keepdims=True)))[:, 0]
    want = (lse - z[np.arange(9), tgt.numpy()]).sum() / 3.0
    assert abs(float(loss) - want) < 1e-12 * max(1.0, abs(want))


def test_softcap_gradient_finite_differences():
    g = torch.Generator().manual_seed(1)
    h, W = torch.randn(3, 8, generator=g), torch.randn(20, 8, generator=g) * 3
    tgt = torch.tensor([1, 7, 19])
    _, grad = LR.full_ce(h, W, tgt, 5.0)
    eps = 1e-6
    num = torch.zeros_like(grad)
    for i in range(3):
        for j in range(8):
            hp, hm = h.double().clone(), h.double().clone()
            hp[i, j] += eps
            hm[i, j] -= eps
            num[i, j] = (LR.full_ce(hp, W, tgt, 5.0)[0] - LR.full_ce(hm, W, tgt, 5.0)[0]) / (2 * eps)
    assert torch.allclose(grad, num, rtol=1e-6, atol=1e-8)


def test_ce_entry_points_reject_bad_arguments():
    from smel import _lib
    L = _lib.load()
    fake = ctypes.c_void_p(1 << 20)   # never dereferenced
    EINVAL = -1
    cu = L.smel_ce_chunk_update
    assert cu(fake, 4, 0, 0, 0, fake, 0.0, 0, 1, fake, fake, fake, fake, fake, 1, fake, None) == EINVAL  # vc 0
    assert cu(fake, 4, 8, 4, 0, fake, 0.0, 0, 1, fake, fake, fake, fake, fake, 1, fake, None) == EINVAL  # ld < vc
    assert cu(fake, 4, 8, 8, 0, fake, 0.0, 3, 1, fake, fake, fake, fake, fake, 1, fake, None) == EINVAL  # dtype
    assert cu(fake, 4, 8, 8, 0, fake, 0.0, 0, 1, fake, fake, fake, fake, None, 1, fake, None) == EINVAL  # no p
    assert cu(fake, 4, 8, 8, 0, fake, 0.0, 0, 1, fake, fake, fake, fake, fake, 3, fake, None) == EINVAL  # 3 parts
    assert cu(fake, 0, 8, 8, 0, fake, 0.0, 0, 1, fake, fake, fake, fake, fake, 2, fake, None) == 0       # no rows
    assert L.smel_ce_acc_update(fake, fake, None, 1, 4, 8, 0, None) == EINVAL
    assert L.smel_ce_acc_update(fake, fake, fake, 1, 4, 0, 0, None) == EINVAL
    assert L.smel_ce_acc_update(fake, fake, fake, 0, 4, 8, 0, None) == EINVAL
