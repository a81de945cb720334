"""Pin the oracle's layer frontends (short convolution + SiLU, gated RMS norm) by independent
formulations: torch's grouped conv1d, a per-element brute-force loop, autograd, and closed
forms.  CPU only."""
import pytest
import torch
import torch.nn.functional as F

from oracle import kdn_oracle as ko


@pytest.fixture(autouse=True)
def _fp64_default():
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def _brute_conv(x, w):
    B, T, D = x.shape
    y = torch.zeros(B, T, D)
    for b in range(B):
        for t in range(T):
            for d in range(D):
                acc = 0.0
                for j in range(4):
                    s = t - 3 + j
                    if s >= 0:
                        acc += float(w[d, j]) * float(x[b, s, d])
                y[b, t, d] = acc / (1.0 + torch.exp(torch.tensor(-acc))) if acc > -700 else 0.0
    return y


def test_short_conv_matches_conv1d_and_brute_force():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 7, 5, generator=g)
    w = torch.randn(5, 4, generator=g)
    y = ko.short_conv_silu(x, w)
    assert torch.allclose(y, ko.short_conv_silu_conv1d(x, w), atol=1e-13, rtol=0)
    assert torch.allclose(y, _brute_conv(x, w), atol=1e-12, rtol=0)


def test_short_conv_first_tokens_and_single_token():
    """Zero history: y_0 = silu(w_3 x_0), y_1 = silu(w_2 x_0 + w_3 x_1); T = 1 is the reference's
    one-token update with a zero cache."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, 3, 4, generator=g)
    w = torch.randn(4, 4, generator=g)
    y = ko.short_conv_silu(x, w)
    assert torch.allclose(y[0, 0], F.silu(w[:, 3] * x[0, 0]))
    assert torch.allclose(y[0, 1], F.silu(w[:, 2] * x[0, 0] + w[:, 3] * x[0, 1]))
    assert torch.allclose(ko.short_conv_silu(x[:, :1], w)[0, 0], F.silu(w[:, 3] * x[0, 0]))


def test_qkv_conv_backward_rule_is_the_exact_gradient():
    """Without the preactivation rounding, the reference kernel's backward rule equals autograd."""
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 11, 6, generator=g, requires_grad=True)
    w = torch.randn(6, 4, generator=g, requires_grad=True)
    dy = torch.randn(2, 11, 6, generator=g)
    dx_ref, dw_ref = torch.autograd.grad((ko.short_conv_silu(x, w) * dy).sum(), (x, w))
    dx, dw = ko.qkv_conv_backward(x.detach(), w.detach(), dy)
    assert torch.allclose(dx, dx_ref, atol=1e-12, rtol=0)
    assert torch.allclose(dw, dw_ref, atol=1e-12, rtol=0)


def test_qkv_conv_backward_rounding_moves_only_silu_prime():
    """With a bf16 preactivation buffer the rule differs from the exact gradient by bf16's
    relative rounding of y inside silu' only (a small, bounded perturbation)."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, 40, 8, generator=g)
    w = torch.randn(8, 4, generator=g)
    dy = torch.randn(1, 40, 8, generator=g)
    dx0, dw0 = ko.qkv_conv_backward(x, w, dy)
    dx1, dw1 = ko.qkv_conv_backward(x, w, dy, raw_dtype=torch.bfloat16)
    assert not torch.equal(dx0, dx1)
    assert float((dx1 - dx0).abs().max() / dx0.abs().max()) < 1e-2
    assert float((dw1 - dw0).abs().max() / dw0.abs().max()) < 1e-2


def test_short_conv_gradcheck():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(1, 6, 3, generator=g, requires_grad=True)
    w = torch.randn(3, 4, generator=g, requires_grad=True)
    assert torch.autograd.gradcheck(ko.short_conv_silu, (x, w))


@pytest.mark.parametrize("activation", ["sigmoid", "swish"])
def test_rms_norm_gated_closed_form_and_gradcheck(activation):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 4, 16, generator=g, requires_grad=True)
    gate = torch.randn(3, 4, 16, generator=g, requires_grad=True)
    w = torch.randn(16, generator=g, requires_grad=True)
    y = ko.rms_norm_gated(x, gate, w, eps=1e-5, activation=activation)
    # row by row: y = x / sqrt(mean(x^2) + eps) * w * act(g)
    for b in range(3):
        for t in range(4):
            xr, gr = x[b, t].detach(), gate[b, t].detach()
            act = torch.sigmoid(gr) if activation == "sigmoid" else gr * torch.sigmoid(gr)
            ref = xr / torch.sqrt((xr * xr).sum() / 16 + 1e-5) * w.detach() * act
            assert torch.allclose(y[b, t].detach(), ref, atol=1e-13, rtol=0)
    # a constant row normalises to +-1 (eps aside): x = c -> y = c / sqrt(c^2 + eps) w act(g)
    c = torch.full((1, 1, 16), 3.0)
    yc = ko.rms_norm_gated(c, torch.zeros(1, 1, 16), torch.ones(16), eps=0.0, activation="sigmoid")
    assert torch.allclose(yc, torch.full((1, 1, 16), 0.5))
    assert torch.autograd.gradcheck(lambda a, b, c_: ko.rms_norm_gated(a, b, c_, 1e-5, activation), (x, gate, w))


def test_layer_frontend_wrappers_reject_bad_arguments():
    """Argument checks of the product wrappers fire before any device work (reference
    iso_kdn_chunk.py:257-283)."""
    from lit_gpt.kdn_ops import short_conv, gated_norm
    x = torch.zeros(1, 4, 9, dtype=torch.float32)
    with pytest.raises(ValueError):
        short_conv.qkv_causal_conv1d(x, torch.zeros(9, 3))  # width must be 4
    with pytest.raises(ValueError):
        short_conv.qkv_causal_conv1d(torch.zeros(1, 4, 8), torch.zeros(8, 4))  # not a multiple of 3
    with pytest.raises(NotImplementedError):
        short_conv.causal_conv1d(torch.zeros(1, 4, 8), torch.zeros(8, 4), bias=torch.zeros(8))
    with pytest.raises(ValueError):
        gated_norm.rms_norm_gated(torch.zeros(2, 16), torch.zeros(2, 8), torch.ones(16))
    with pytest.raises(NotImplementedError):
        gated_norm.FusedRMSNormGated(16, activation="relu")
