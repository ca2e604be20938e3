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
    """Host-side checks of include/smel_loss.h: bad sizes, dtypes and layouts are refused before any launch."""
    from smel import _lib
    L = _lib.load()
    fake = ctypes.c_void_p(1 << 20)   # 16-byte aligned, never dereferenced
    EINVAL, EUNSUP = -1, -2
    lg = L.smel_ce_logits   # W ldw vc v0 h ldh n H tgt cap dtype P ldp win_e win_s ldn tz td stream
    ok = (fake, 64, 300, 0, fake, 64, 4, 64, fake, 0.0, 0, fake, 512, fake, fake, 4, fake, fake)
    assert lg(*ok[:10], 3, *ok[11:], None) == EINVAL                       # dtype
    assert lg(*ok[:2], 0, *ok[3:], None) == EINVAL                          # empty chunk
    assert lg(*ok[:7], 12, *ok[8:], None) == EUNSUP                         # 24-byte bf16 rows
    assert lg(*ok[:12], 300, *ok[13:], None) == EINVAL                      # softmax rows shorter than 512
    assert lg(*ok[:15], 3, *ok[16:], None) == EINVAL                        # statistics pitch below n
    assert lg(*ok[:6], 0, *ok[7:], None) == 0                               # no rows: nothing to do
    gr = L.smel_ce_grad     # WT ldwt H P ldp vc shift ldn r n dtype chunk acc part stream
    assert gr(fake, 512, 66, fake, 512, 300, fake, 4, fake, 4, 0, 0, fake, fake, None) == EUNSUP   # H % 4
    assert gr(fake, 512, 64, None, 512, 300, fake, 4, fake, 4, 0, 0, fake, fake, None) == EINVAL   # no softmax terms
    assert gr(fake, 256, 64, fake, 512, 300, fake, 4, fake, 4, 0, 0, fake, fake, None) == EUNSUP  # head rows short
    assert gr(fake, 512, 64, fake, 512, 300, fake, 4, None, 4, 0, 1, fake, fake, None) == EINVAL   # no rescale
    assert gr(fake, 512, 64, fake, 512, 300, fake, 4, fake, 4, 0, 0, fake, None, None) == EINVAL   # no partials
    assert L.smel_ce_stats(fake, fake, 0, 4, 4, fake, fake, fake, fake, None) == EINVAL         # no windows
    assert L.smel_ce_finish(fake, fake, fake, fake, None, None, None, 0, None, fake, 10, 4, 64, 5, 1.0, None, 0, 0,
                            fake, None) == EINVAL                                               # dtype
    assert L.smel_ce_transpose(fake, 4, 64, 32, fake, 8, 0, None) == EINVAL                    # pitch < columns
    assert L.smel_ce_scale(fake, 8, 3, fake, None) == EINVAL
    assert L.smel_ce_loss_sum(fake, 4, 1.0, 0, None, None) == EINVAL
