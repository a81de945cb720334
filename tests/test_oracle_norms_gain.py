"""Pin the oracle functions that no golden vector covers directly.

* ``l2norm_fla`` (FLA l2norm_fwd, x * rsqrt(sum x^2 + 1e-6), iso_kdn_chunk.py:2203-2204): unit norm
  for rows with sum x^2 >> eps, a zero row maps to zero, invariance to positive scaling of large
  rows, and the eps inside the square root.  The last check separates the plausible variants: at
  x = c e_1 with c^2 = eps the result is 1/sqrt(2) e_1, where x / (|x| + eps) gives ~0.999 and
  x / max(|x|, eps) gives 1.
* ``diag_normalize`` (x / max(||x||, 1e-12), diag_kdn_chunk.py:194-232) against
  ``torch.nn.functional.normalize(x, dim=-1, eps=1e-12)``, a library routine with that definition,
  including zero rows and rows below the floor.
* ``iso_gain_unit_key`` (the production iso gain, iso_kdn_chunk.py:1586-1594) against the closed
  form z = a p + w, beta = z / (r + z), p' = r z / (r + s z), and against the golden-pinned
  ``iso_gain_tokenwise`` on random unit keys of width K with a = mean alpha^2; gradients included.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import kdn_oracle as ko


def _g(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------------------- l2norm_fla

def test_l2norm_fla_unit_norm_for_large_rows():
    x = torch.randn(5, 7, 128, generator=_g(0), dtype=torch.float64)
    y = ko.l2norm_fla(x)
    n = y.norm(dim=-1)
    # |y| = |x| / sqrt(|x|^2 + eps): 1 to within eps / (2 |x|^2) ~ 4e-9 here
    assert float((n - 1).abs().max()) < 1e-7
    # the direction is x's
    cos = (y * x).sum(-1) / (y.norm(dim=-1) * x.norm(dim=-1))
    assert float((cos - 1).abs().max()) < 1e-12


def test_l2norm_fla_zero_row_maps_to_zero():
    x = torch.zeros(3, 64, dtype=torch.float64)
    x[1] = torch.randn(64, generator=_g(1), dtype=torch.float64)
    y = ko.l2norm_fla(x)
    assert torch.equal(y[0], torch.zeros(64, dtype=torch.float64))
    assert torch.equal(y[2], torch.zeros(64, dtype=torch.float64))
    assert torch.isfinite(y).all()


@pytest.mark.parametrize("c", [0.25, 3.0, 100.0])
def test_l2norm_fla_scale_invariance(c):
    x = torch.randn(4, 128, generator=_g(2), dtype=torch.float64)
    torch.testing.assert_close(ko.l2norm_fla(c * x), ko.l2norm_fla(x), rtol=1e-7, atol=1e-7)


def test_l2norm_fla_eps_inside_square_root():
    eps = 1e-6
    c = math.sqrt(eps)
    x = torch.zeros(2, 16, dtype=torch.float64)
    x[0, 0] = c
    x[1, 3] = -2 * c  # |x|^2 = 4 eps -> 2c / sqrt(5 eps) = 2 / sqrt(5)
    y = ko.l2norm_fla(x)
    assert abs(float(y[0, 0]) - 1 / math.sqrt(2)) < 1e-12
    assert abs(float(y[1, 3]) + 2 / math.sqrt(5)) < 1e-12
    # not the alternatives a transcription could produce
    assert abs(float(y[0, 0]) - c / (c + eps)) > 0.2
    assert abs(float(y[0, 0]) - 1.0) > 0.2


def test_l2norm_fla_gradient_is_projection_for_large_rows():
    """d/dx of x/|x| is (I - y y^T)/|x|: the gradient is orthogonal to y."""
    x = torch.randn(3, 32, generator=_g(3), dtype=torch.float64).requires_grad_(True)
    dy = torch.randn(3, 32, generator=_g(4), dtype=torch.float64)
    y = ko.l2norm_fla(x)
    (dx,) = torch.autograd.grad((y * dy).sum(), x)
    yd = y.detach()
    expect = (dy - yd * (yd * dy).sum(-1, keepdim=True)) / x.detach().norm(dim=-1, keepdim=True)
    torch.testing.assert_close(dx, expect, rtol=1e-6, atol=1e-9)


# ---------------------------------------------------------------------------- diag_normalize

@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_diag_normalize_equals_torch_normalize(dtype):
    x = torch.randn(6, 9, 128, generator=_g(5), dtype=torch.float64).to(dtype)
    x[0, 0] = 0.0                      # zero row
    x[1, 2] = 1e-15                    # norm below the 1e-12 floor
    x[2, 3] = 1e-11 * torch.randn(128, generator=_g(6), dtype=torch.float64).to(dtype)
    y = ko.diag_normalize(x)
    ref = F.normalize(x, dim=-1, eps=1e-12)
    torch.testing.assert_close(y, ref, rtol=2e-7 if dtype == torch.float32 else 1e-15, atol=0.0)
    assert torch.equal(y[0, 0], torch.zeros_like(y[0, 0]))


def test_diag_normalize_gradient_equals_torch_normalize():
    x = torch.randn(4, 64, generator=_g(7), dtype=torch.float64)
    x[1] = 0.0
    dy = torch.randn(4, 64, generator=_g(8), dtype=torch.float64)
    a = x.clone().requires_grad_(True)
    b = x.clone().requires_grad_(True)
    (ga,) = torch.autograd.grad((ko.diag_normalize(a) * dy).sum(), a)
    (gb,) = torch.autograd.grad((F.normalize(b, dim=-1, eps=1e-12) * dy).sum(), b)
    torch.testing.assert_close(ga, gb, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------- unit-key iso gain

def _gain_inputs(seed, B, T, H):
    g = _g(seed)
    a = torch.sigmoid(2 + 0.5 * torch.randn(B, T, H, generator=g, dtype=torch.float64)) ** 2
    omega = F.softplus(torch.randn(B, T, H, generator=g, dtype=torch.float64))
    r = 0.01 + F.softplus(torch.randn(B, T, H, generator=g, dtype=torch.float64))
    mu = 0.5 + torch.rand(H, generator=g, dtype=torch.float64)
    return a, omega, r, mu


@pytest.mark.parametrize("s", [1.0, 0.5])
def test_unit_key_gain_closed_form(s):
    B, T, H = 2, 40, 3
    a, omega, r, mu = _gain_inputs(9, B, T, H)
    beta, c = ko.iso_gain_unit_key(a, omega, r, mu, posterior_scale=s, output_final_state=True)
    p = (1.0 / mu).view(1, H).expand(B, H)
    for t in range(T):
        z = a[:, t] * p + omega[:, t]
        torch.testing.assert_close(beta[:, t], z / (r[:, t] + z), rtol=1e-13, atol=0.0)
        p = r[:, t] * z / (r[:, t] + s * z)
    torch.testing.assert_close(c, 1.0 / p, rtol=1e-13, atol=0.0)


@pytest.mark.parametrize("info_scale,K", [(None, 16), (8.0, 16), (None, 64)])
def test_unit_key_gain_equals_tokenwise_on_unit_keys(info_scale, K):
    """Random unit keys of width K and random per-channel alpha: the tokenwise gain (golden-pinned)
    depends on them only through |k|^2 = 1 and a = mean alpha^2."""
    B, T, H = 2, 33, 2
    g = _g(10 + K)
    k = torch.randn(B, T, H, K, generator=g, dtype=torch.float64)
    k = k / k.norm(dim=-1, keepdim=True)
    alpha = torch.sigmoid(2 + 0.5 * torch.randn(B, T, H, K, generator=g, dtype=torch.float64))
    omega = F.softplus(torch.randn(B, T, H, generator=g, dtype=torch.float64))
    r = 0.01 + F.softplus(torch.randn(B, T, H, generator=g, dtype=torch.float64))
    mu = 0.5 + torch.rand(B, H, generator=g, dtype=torch.float64)
    leaves = [x.clone().requires_grad_(True) for x in (alpha, omega, r, mu)]
    beta_ref, c_ref = ko.iso_gain_tokenwise(k, leaves[0], leaves[1], leaves[2], info_scale=info_scale,
                                            initial_precision=leaves[3], output_final_state=True)
    s = (K if info_scale is None else info_scale) / K
    a = leaves[0].square().mean(-1)
    beta, c = ko.iso_gain_unit_key(a, leaves[1], leaves[2], leaves[3], posterior_scale=s, output_final_state=True)
    torch.testing.assert_close(beta, beta_ref, rtol=1e-12, atol=1e-14)
    torch.testing.assert_close(c, c_ref, rtol=1e-12, atol=1e-14)
    w = torch.randn(B, T, H, generator=g, dtype=torch.float64)
    wc = torch.randn(B, H, generator=g, dtype=torch.float64)
    g_ref = torch.autograd.grad((beta_ref * w).sum() + (c_ref * wc).sum(), leaves, retain_graph=True)
    g_unit = torch.autograd.grad((beta * w).sum() + (c * wc).sum(), leaves)
    for x, y in zip(g_unit, g_ref):
        torch.testing.assert_close(x, y, rtol=1e-10, atol=1e-12)


def test_iso_mixer_uses_unit_key_gain():
    """The oracle mixer's beta is the unit-key gain of its own frontend scalars: with q = k (so the
    memory readout is easy to predict at T = 1) the first output is scale * beta_0 * v_0 (|k| = 1)."""
    B, T, H, K = 1, 1, 2, 16
    g = _g(11)
    q = torch.randn(B, T, H, K, generator=g, dtype=torch.float64)
    v = torch.randn(B, T, H, K, generator=g, dtype=torch.float64)
    g_raw = torch.randn(B, T, H, K, generator=g, dtype=torch.float64)
    orr = torch.randn(B, T, 2 * H, generator=g, dtype=torch.float64)
    zeros = torch.zeros(H, dtype=torch.float64)
    mu_p = torch.randn(H, generator=g, dtype=torch.float64)
    o = ko.iso_mixer(q, q, v, g_raw, orr, zeros, zeros, zeros, torch.zeros(H * K, dtype=torch.float64), mu_p)
    _g_log, _gc, a, omega, r, mu = ko.iso_gate_frontend(g_raw, orr, zeros, zeros, zeros,
                                                        torch.zeros(H * K, dtype=torch.float64), mu_p)
    beta, _ = ko.iso_gain_unit_key(a, omega, r, mu)
    qn = ko.l2norm_fla(q)
    expect = K ** -0.5 * beta[..., None] * (qn * qn).sum(-1, keepdim=True) * v
    torch.testing.assert_close(o, expect, rtol=1e-12, atol=1e-14)
