"""GPU parity of the layer frontends (kdn_short_conv_* and kdn_rms_norm_gated_* through the
C ABI) against the CPU oracle.

* Short convolution + SiLU: forward and dx/dweight against autograd of the fp64 oracle, and the
  packed q|k|v backward against the reference kernel's rule (bf16 preactivation buffer,
  ``ko.qkv_conv_backward``).  fp32 inputs at 1e-5, bf16 at 2e-2 (bf16 outputs / gradients).
* Gated RMS norm (sigmoid and swish): y, dx, dg, dweight at 1e-5 (fp32) and 2e-2 (bf16).
* Edge cases: T = 1 and T < 4 (zero history), a 64-token block boundary, packed strided
  views, determinism of the weight-gradient sums.
"""
import pytest
import torch

from gpu_util import gpu_or_skip, log, rel
from oracle import kdn_oracle as ko

pytestmark = pytest.mark.gpu
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


def _check(name, got, ref, tol):
    r = rel(got, ref)
    log(f"  {name}: rel err {r:.3e} (tol {tol:g})")
    assert r <= tol, f"{name}: {r:.3e} > {tol}"


@pytest.mark.parametrize("B,T,D,dtype", [(2, 150, 64, torch.float32), (2, 150, 64, torch.bfloat16),
                                         (1, 1, 16, torch.float32), (3, 3, 8, torch.bfloat16),
                                         (1, 300, 256, torch.bfloat16)])
def test_short_conv_matches_oracle(B, T, D, dtype):
    dev = gpu_or_skip()
    from lit_gpt.kdn_ops.short_conv import causal_conv1d
    log(f"case short conv B={B} T={T} D={D} {dtype}")
    g = torch.Generator().manual_seed(T + D)
    x = torch.randn(B, T, D, generator=g).to(dtype)
    w = (0.5 * torch.randn(D, 4, generator=g)).to(dtype)
    dy = torch.randn(B, T, D, generator=g).to(dtype)
    xd, wd = x.double().requires_grad_(True), w.double().requires_grad_(True)
    y_ref = ko.short_conv_silu(xd, wd)
    dx_ref, dw_ref = torch.autograd.grad((y_ref * dy.double()).sum(), (xd, wd))
    xg, wg = x.to(dev).requires_grad_(True), w.to(dev).requires_grad_(True)
    y, state = causal_conv1d(xg, wg, activation="silu")
    assert state is None and y.dtype == dtype
    dx, dw = torch.autograd.grad(y, (xg, wg), dy.to(dev))
    torch.cuda.synchronize()
    tol = TOL[dtype]
    _check("y", y, y_ref, tol)
    _check("dx", dx, dx_ref, tol)
    _check("dweight", dw, dw_ref, tol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_qkv_causal_conv1d_matches_reference_rule(dtype):
    dev = gpu_or_skip()
    from lit_gpt.kdn_ops.short_conv import qkv_causal_conv1d
    B, T, D = 2, 200, 128  # 200 tokens: four 64-token partial-sum blocks, the last partial
    log(f"case packed qkv conv B={B} T={T} D={D} {dtype}")
    g = torch.Generator().manual_seed(7)
    x = torch.randn(B, T, 3 * D, generator=g).to(dtype)
    w = (0.5 * torch.randn(3 * D, 4, generator=g)).to(dtype)
    dys = [torch.randn(B, T, D, generator=g).to(dtype) for _ in range(3)]
    xg, wg = x.to(dev).requires_grad_(True), w.to(dev).requires_grad_(True)
    outs = qkv_causal_conv1d(xg, wg)
    dx, dw = torch.autograd.grad(outs, (xg, wg), [d.to(dev) for d in dys])
    torch.cuda.synchronize()
    tol = TOL[dtype]
    raw = torch.bfloat16 if dtype == torch.bfloat16 else None
    for gi, name in enumerate("qkv"):
        xs, ws = x[..., gi * D:(gi + 1) * D].double(), w[gi * D:(gi + 1) * D].double()
        _check(f"{name}", outs[gi], ko.short_conv_silu(xs, ws), tol)
        dx_ref, dw_ref = ko.qkv_conv_backward(xs, ws, dys[gi].double(), raw_dtype=raw)
        _check(f"d{name} x", dx[..., gi * D:(gi + 1) * D], dx_ref, tol)
        _check(f"d{name} weight", dw[gi * D:(gi + 1) * D], dw_ref, tol)
    # the weight-gradient sums are in a fixed order: a second backward is bit-identical
    dx2, dw2 = torch.autograd.grad(qkv_causal_conv1d(xg, wg), (xg, wg), [d.to(dev) for d in dys])
    assert torch.equal(dw, dw2) and torch.equal(dx, dx2)


@pytest.mark.parametrize("shape,D,dtype,act", [((2, 100, 4), 128, torch.bfloat16, "sigmoid"),
                                               ((3, 7, 2), 64, torch.float32, "sigmoid"),
                                               ((2, 33, 3), 128, torch.float32, "swish"),
                                               ((1, 1, 1), 128, torch.bfloat16, "sigmoid")])
def test_rms_norm_gated_matches_oracle(shape, D, dtype, act):
    dev = gpu_or_skip()
    from lit_gpt.kdn_ops.gated_norm import FusedRMSNormGated
    log(f"case gated rms norm {shape} D={D} {dtype} {act}")
    g = torch.Generator().manual_seed(D + len(shape))
    x = torch.randn(*shape, D, generator=g).to(dtype)
    gate = torch.randn(*shape, D, generator=g).to(dtype)
    w = 1.0 + 0.1 * torch.randn(D, generator=g)
    dy = torch.randn(*shape, D, generator=g).to(dtype)
    xd, gd, wd = (t.double().requires_grad_(True) for t in (x, gate, w))
    y_ref = ko.rms_norm_gated(xd, gd, wd, eps=1e-5, activation=act)
    dx_ref, dg_ref, dw_ref = torch.autograd.grad((y_ref * dy.double()).sum(), (xd, gd, wd))
    norm = FusedRMSNormGated(D, activation=act, eps=1e-5).to(dev)
    with torch.no_grad():
        norm.weight.copy_(w)
    xg, gg = x.to(dev).requires_grad_(True), gate.to(dev).requires_grad_(True)
    y = norm(xg, gg)
    assert y.dtype == dtype and y.shape == x.shape
    dx, dgate, dw = torch.autograd.grad(y, (xg, gg, norm.weight), dy.to(dev))
    torch.cuda.synchronize()
    tol = TOL[dtype]
    _check("y", y, y_ref, tol)
    _check("dx", dx, dx_ref, tol)
    _check("dg", dgate, dg_ref, tol)
    _check("dweight", dw, dw_ref, tol)
