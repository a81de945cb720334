"""Gated RMS norm of the KDN mixer output (the layers' ``o_norm``).

Drop-in for FLA's ``FusedRMSNormGated`` / ``rms_norm_gated`` as the reference layers use it
(ngocbh/kalman-delta-networks ``lit_gpt/iso_kdn.py:192-196,305-312``,
``lit_gpt/diag_kdn.py:216-219,346``):

    y = x * rsqrt(mean(x^2, -1) + eps) * weight * act(g)

with act = sigmoid (``activation="sigmoid"``, the layers' choice) or g * sigmoid(g)
(``"swish"`` / ``"silu"``).  f32 arithmetic; y in x's dtype; the backward returns dx (x's
dtype), dg (g's dtype) and dweight (weight's dtype, a fixed-order sum over rows).  Residual /
prenorm / bias variants of the FLA module are not used by the layers and are rejected.
All arithmetic runs in ``libkdn_hip.so``.
"""
from __future__ import annotations

import torch
from torch import nn
from torch.autograd.function import once_differentiable

from . import _lib

_ACT = {"sigmoid": 0, "swish": 1, "silu": 1}


def _flat(t, D):
    return t.reshape(-1, D)


class _RMSNormGatedFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, g, weight, eps, act):
        D = x.shape[-1]
        xf, gf = _flat(x, D), _flat(g, D)
        rows = xf.shape[0]
        y = torch.empty_like(xf)
        rstd = torch.empty(rows, device=x.device, dtype=torch.float32)
        with torch.cuda.device(x.device):
            _lib.call("kdn_rms_norm_gated_fwd", _lib.ptr(xf), _lib.is_bf16(xf), _lib.ptr(gf), _lib.is_bf16(gf),
                      _lib.ptr(weight), _lib.is_bf16(weight), rows, D, float(eps), act, _lib.ptr(y), _lib.ptr(rstd),
                      _lib.stream_of(x), tag="rms_norm_gated_fwd")
        ctx.save_for_backward(xf, gf, weight, rstd)
        ctx.act = act
        ctx.shape = x.shape
        ctx.set_materialize_grads(False)
        return y.view(x.shape)

    @staticmethod
    @once_differentiable
    def backward(ctx, dy):
        if dy is None:
            return None, None, None, None, None
        xf, gf, weight, rstd = ctx.saved_tensors
        rows, D = xf.shape
        dyf = _flat(dy.to(xf.dtype).contiguous(), D)
        dx = torch.empty_like(xf) if ctx.needs_input_grad[0] else None
        dg = torch.empty_like(gf) if ctx.needs_input_grad[1] else None
        dw = torch.empty_like(weight) if ctx.needs_input_grad[2] else None
        ws_bytes = _lib.size("kdn_rms_norm_gated_bwd_workspace_size", rows, D) if dw is not None else 0
        ws = torch.empty(max(ws_bytes // 4, 1), device=xf.device, dtype=torch.float32) if dw is not None else None
        with torch.cuda.device(xf.device):
            _lib.call("kdn_rms_norm_gated_bwd", _lib.ptr(xf), _lib.is_bf16(xf), _lib.ptr(gf), _lib.is_bf16(gf),
                      _lib.ptr(weight), _lib.is_bf16(weight), _lib.ptr(rstd), _lib.ptr(dyf), rows, D, ctx.act,
                      _lib.ptr(dx), _lib.ptr(dg), _lib.ptr(dw), _lib.ptr(ws), ws_bytes, _lib.stream_of(xf),
                      tag="rms_norm_gated_bwd")
        shape = ctx.shape
        return (dx.view(shape) if dx is not None else None, dg.view(shape) if dg is not None else None, dw, None,
                None)


def rms_norm_gated(x, g, weight, bias=None, activation="swish", residual=None, prenorm=False,
                   residual_in_fp32=False, eps=1e-6):
    """FLA ``rms_norm_gated`` for the configuration the layers use (no bias, no residual)."""
    if bias is not None or residual is not None or prenorm:
        raise NotImplementedError("bias / residual / prenorm variants are not supported")
    if activation not in _ACT:
        raise NotImplementedError(f"activation {activation!r} is not supported")
    if not isinstance(x, torch.Tensor) or not isinstance(g, torch.Tensor):
        raise TypeError("x and g must be tensors")
    if x.shape != g.shape:
        raise ValueError(f"x and g must have the same shape, got {tuple(x.shape)} and {tuple(g.shape)}")
    D = x.shape[-1]
    if weight is None or weight.shape != (D,):
        raise ValueError(f"weight must have shape ({D},)")
    if D % 8 or (D // 8) & (D // 8 - 1) or D // 8 > 64:
        raise ValueError("the normalised dimension must be 8 * 2^n <= 512")
    for name, t in (("x", x), ("g", g), ("weight", weight)):
        if t.dtype not in (torch.bfloat16, torch.float32):
            raise TypeError(f"{name} must be bfloat16 or float32")
    _lib.require_device(x, g, weight)
    x, g, weight = x.contiguous(), g.contiguous(), weight.contiguous()
    return _RMSNormGatedFunction.apply(x, g, weight, float(eps), _ACT[activation])


class FusedRMSNormGated(nn.Module):
    """FLA ``FusedRMSNormGated(hidden_size, elementwise_affine=True, eps=1e-5, activation="swish")``;
    ``forward(x, g)`` normalises over the last dimension (``hidden_size``)."""

    def __init__(self, hidden_size: int, elementwise_affine: bool = True, eps: float = 1e-5,
                 activation: str = "swish", device=None, dtype=None):
        super().__init__()
        if activation not in _ACT:
            raise NotImplementedError(f"activation {activation!r} is not supported")
        self.hidden_size = hidden_size
        self.elementwise_affine = elementwise_affine
        self.eps = eps
        self.activation = activation
        if elementwise_affine:
            self.weight = nn.Parameter(torch.ones(hidden_size, device=device, dtype=dtype))
        else:
            self.register_parameter("weight", None)

    def forward(self, x, g, residual=None, prenorm=False, residual_in_fp32=False):
        weight = self.weight if self.weight is not None else torch.ones(self.hidden_size, device=x.device)
        return rms_norm_gated(x, g, weight, activation=self.activation, residual=residual, prenorm=prenorm,
                              residual_in_fp32=residual_in_fp32, eps=self.eps)

    def extra_repr(self) -> str:
        return f"{self.hidden_size}, eps={self.eps}, activation={self.activation}"


__all__ = ("rms_norm_gated", "FusedRMSNormGated")
