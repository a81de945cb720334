"""Block RMS norm of the model (``FusedRMSNorm``), on the HIP library.

Mirrors ``lit_gpt/rmsnorm.py:1182-1216`` of the reference (ngocbh/kalman-delta-networks) for the
configuration the KDN models use: no residual, no dropout, no zero-centred weight;
y = x rsqrt(mean(x^2) + eps) * weight in f32, returned in x's dtype.
"""
from __future__ import annotations

import torch
from torch import nn
from torch.autograd.function import once_differentiable

from .kdn_ops import _lib


class _RMSNormFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, eps):
        D = x.shape[-1]
        xf = x.reshape(-1, D)
        rows = xf.shape[0]
        y = torch.empty_like(xf)
        rstd = torch.empty(rows, device=x.device, dtype=torch.float32)
        with torch.cuda.device(x.device):
            _lib.call("kdn_rms_norm_fwd", _lib.ptr(xf), _lib.is_bf16(xf), _lib.ptr(weight), _lib.is_bf16(weight),
                      rows, D, float(eps), _lib.ptr(y), _lib.ptr(rstd), _lib.stream_of(x), tag="rms_norm_fwd")
        ctx.save_for_backward(xf, weight, rstd)
        ctx.shape = x.shape
        return y.view(x.shape)

    @staticmethod
    @once_differentiable
    def backward(ctx, dy):
        xf, weight, rstd = ctx.saved_tensors
        rows, D = xf.shape
        dyf = dy.to(xf.dtype).reshape(-1, D).contiguous()
        dx = torch.empty_like(xf) if ctx.needs_input_grad[0] else None
        dw = torch.empty_like(weight) if ctx.needs_input_grad[1] else None
        ws_bytes = _lib.size("kdn_rms_norm_bwd_workspace_size", rows, D) if dw is not None else 0
        ws = torch.empty(max(ws_bytes // 4, 1), device=xf.device, dtype=torch.float32) if dw is not None else None
        with torch.cuda.device(xf.device):
            _lib.call("kdn_rms_norm_bwd", _lib.ptr(xf), _lib.is_bf16(xf), _lib.ptr(weight), _lib.is_bf16(weight),
                      _lib.ptr(rstd), _lib.ptr(dyf), rows, D, _lib.ptr(dx), _lib.ptr(dw), _lib.ptr(ws), ws_bytes,
                      _lib.stream_of(xf), tag="rms_norm_bwd")
        return (dx.view(ctx.shape) if dx is not None else None), dw, None


def rms_norm_fn(x, weight, bias=None, residual=None, eps=1e-6, dropout_p=0.0, prenorm=False,
                residual_in_fp32=False, zero_centered_weight=False):
    """The reference's ``rms_norm_fn`` for the plain case (no bias / residual / dropout)."""
    if bias is not None or residual is not None or dropout_p or prenorm or zero_centered_weight:
        raise NotImplementedError("only the plain RMS norm is supported")
    D = x.shape[-1]
    if weight.shape != (D,):
        raise ValueError(f"weight must have shape ({D},)")
    if D % 8 or D > 8192:
        raise ValueError("the normalised dimension must be a multiple of 8 and at most 8192")
    for name, t in (("x", x), ("weight", weight)):
        if t.dtype not in (torch.bfloat16, torch.float32):
            raise TypeError(f"{name} must be bfloat16 or float32")
    _lib.require_device(x, weight)
    return _RMSNormFunction.apply(x.contiguous(), weight.contiguous(), float(eps))


class FusedRMSNorm(nn.Module):
    """``FusedRMSNorm(hidden_size, eps=1e-5)`` (reference rmsnorm.py:1182)."""

    def __init__(self, hidden_size, eps=1e-5, dropout_p=0.0, zero_centered_weight=False, device=None, dtype=None):
        super().__init__()
        if dropout_p or zero_centered_weight:
            raise NotImplementedError("dropout / zero-centred weight are not supported")
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size, device=device, dtype=dtype))
        self.register_parameter("bias", None)

    def forward(self, x, residual=None, prenorm=False, residual_in_fp32=False):
        return rms_norm_fn(x, self.weight, residual=residual, eps=self.eps, prenorm=prenorm,
                           residual_in_fp32=residual_in_fp32)


__all__ = ("FusedRMSNorm", "rms_norm_fn")
