"""Pins the cross-entropy oracle (oracle/xent_oracle.py) on the CPU.

Each check compares it with something it does not restate: torch's own cross_entropy (label
smoothing, ignore_index), torch.logsumexp (z-loss), autograd of that library expression (the
backward), an identity of cross_entropy for labels outside the vocabulary, and the whole
vocabulary against its combined slices.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import xent_oracle as xo


def _data(n=23, C=97, seed=0, ignore_index=-100):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, C, generator=g, dtype=torch.float64) * 3
    y = torch.randint(0, C, (n,), generator=g)
    y[::5] = ignore_index
    return x, y


@pytest.mark.parametrize("smoothing", [0.0, 0.1, 0.7])
@pytest.mark.parametrize("scale", [1.0, 0.37])
@pytest.mark.parametrize("ignore_index", [-100, 3])
def test_forward_matches_torch_cross_entropy(smoothing, scale, ignore_index):
    x, y = _data(ignore_index=ignore_index)
    loss, lse, z = xo.xent_forward(x, y, smoothing=smoothing, logit_scale=scale, ignore_index=ignore_index)
    ref = F.cross_entropy(x * scale, y, label_smoothing=smoothing, ignore_index=ignore_index, reduction="none")
    torch.testing.assert_close(loss, ref, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(lse, torch.logsumexp(x * scale, 1), rtol=1e-12, atol=1e-12)
    assert float(z.abs().max()) == 0.0


def test_z_loss_is_scaled_lse_squared():
    x, y = _data(seed=1)
    zs = 3e-3
    loss, lse, z = xo.xent_forward(x, y, lse_square_scale=zs)
    base, _, _ = xo.xent_forward(x, y)
    want = zs * torch.logsumexp(x, 1) ** 2
    want[y == -100] = 0
    torch.testing.assert_close(z, want, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(loss - base, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("smoothing", [0.0, 0.2])
@pytest.mark.parametrize("zs", [0.0, 1e-2])
@pytest.mark.parametrize("scale", [1.0, 1.7])
def test_backward_matches_autograd(smoothing, zs, scale):
    x, y = _data(seed=2)
    d = torch.randn(x.shape[0], dtype=torch.float64)
    xr = x.clone().requires_grad_(True)
    s = xr * scale
    ce = F.cross_entropy(s, y, label_smoothing=smoothing, ignore_index=-100, reduction="none")
    zl = torch.where(y == -100, torch.zeros_like(ce), zs * torch.logsumexp(s, 1) ** 2)
    (g,) = torch.autograd.grad(((ce + zl) * d).sum(), xr)
    _, lse, _ = xo.xent_forward(x, y, smoothing=smoothing, logit_scale=scale, lse_square_scale=zs)
    got = xo.xent_backward(d, x, lse, y, smoothing=smoothing, logit_scale=scale, lse_square_scale=zs)
    torch.testing.assert_close(got, g, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("smoothing", [0.0, 0.3])
def test_label_outside_vocabulary(smoothing):
    # no target class: the smoothing term alone, which cross_entropy gives as
    # CE(label_smoothing=s) - (1 - s) CE for any valid label
    x, _ = _data(seed=3)
    n, C = x.shape
    oob = torch.full((n,), C + 5)
    loss, _, _ = xo.xent_forward(x, oob, smoothing=smoothing)
    y0 = torch.zeros(n, dtype=torch.long)
    want = (F.cross_entropy(x, y0, label_smoothing=smoothing, reduction="none")
            - (1 - smoothing) * F.cross_entropy(x, y0, reduction="none"))
    torch.testing.assert_close(loss, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("smoothing", [0.0, 0.25])
@pytest.mark.parametrize("zs", [0.0, 5e-3])
@pytest.mark.parametrize("world", [2, 3])
def test_split_slices_combine_to_whole(smoothing, zs, world):
    x, y = _data(n=31, C=96, seed=4)
    C = x.shape[1]
    w = C // world
    full_loss, full_lse, full_z = xo.xent_forward(x, y, smoothing=smoothing, lse_square_scale=zs)
    losses, lses = [], []
    for r in range(world):
        l, s, _ = xo.xent_forward(x[:, r * w:(r + 1) * w], y, smoothing=smoothing, lse_square_scale=zs,
                                  total_classes=C, class_start_idx=r * w, split=True)
        losses.append(l)
        lses.append(s)
    loss, z, lse = xo.combine_split(losses, lses, y, lse_square_scale=zs)
    torch.testing.assert_close(loss, full_loss, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(z, full_z, rtol=1e-12, atol=1e-12)
    # each slice's backward with the combined lse is the slice of the whole backward
    d = torch.randn(x.shape[0], dtype=torch.float64)
    whole = xo.xent_backward(d, x, full_lse, y, smoothing=smoothing, lse_square_scale=zs)
    for r in range(world):
        part = xo.xent_backward(d, x[:, r * w:(r + 1) * w], lse, y, smoothing=smoothing, lse_square_scale=zs,
                                total_classes=C, class_start_idx=r * w)
        torch.testing.assert_close(part, whole[:, r * w:(r + 1) * w], rtol=1e-12, atol=1e-12)


def test_precomputed_lse_is_used_as_given():
    x, y = _data(seed=5)
    lse = torch.logsumexp(x, 1)
    a, _, _ = xo.xent_forward(x, y)
    b, lb, _ = xo.xent_forward(x, y, precomputed_lse=lse + 1.0)
    torch.testing.assert_close(lb, lse + 1.0)
    keep = y != -100
    torch.testing.assert_close(b[keep], a[keep] + 1.0)
