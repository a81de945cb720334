"""Depthwise causal short convolution with SiLU: the q, k, v producer of the KDN layers.

Drop-in for the two fixed-length entry points the reference layers call
(ngocbh/kalman-delta-networks):

* ``causal_conv1d(x, weight, bias=None, ..., activation="silu")`` — FLA's short convolution as
  ``lit_gpt/diag_kdn.py:75-96`` calls it per tensor (q, k, v separately), returning
  ``(y, None)``;
* ``qkv_causal_conv1d(x, weight)`` — the iso layer's packed q|k|v convolution
  (``lit_gpt/kdn_ops/iso_kdn_chunk.py:280-478``): x [B,T,3D], weight [3D,4] -> (q, k, v), each
  [B,T,D].

Semantics: y[t] = silu(sum_j w[j] x[t-3+j]) per channel, zero history before t = 0, width 4,
no bias, f32 arithmetic rounded to x's dtype.  The packed backward follows the reference's
kernel (``iso_kdn_chunk.py:127-254``): the preactivation is recomputed into x's dtype before
silu' is taken, and the weight gradient is a fixed-order sum of per-(batch, 64-token block)
partials.  The per-tensor backward keeps the recomputed preactivation in f32 (FLA's
backward is not part of the reference tree).  All arithmetic runs in ``libkdn_hip.so``.
"""
from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from . import _lib

GROUPS = 3
KERNEL_WIDTH = 4


def _conv_fwd(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """x [B,T,D] with unit channel stride (a packed-group view is fine), weight [D,4] dense."""
    B, T, D = x.shape
    y = torch.empty((B, T, D), device=x.device, dtype=x.dtype)
    with torch.cuda.device(x.device):
        _lib.call("kdn_short_conv_fwd", _lib.ptr(x), _lib.is_bf16(x), x.stride(0), x.stride(1), _lib.ptr(weight),
                  _lib.is_bf16(weight), B, T, D, KERNEL_WIDTH, _lib.ptr(y), y.stride(0), y.stride(1),
                  _lib.stream_of(x), tag="short_conv_fwd")
    return y


def _conv_bwd(x, weight, dy, dx, dweight, *, round_preactivation: bool):
    """Writes dx (a [B,T,D] view, unit channel stride) and dweight ([D,4]) for one group."""
    B, T, D = x.shape
    ws_bytes = _lib.size("kdn_short_conv_bwd_workspace_size", B, T, D) if dweight is not None else 0
    ws = torch.empty(max(ws_bytes // 4, 1), device=x.device, dtype=torch.float32) if dweight is not None else None
    with torch.cuda.device(x.device):
        _lib.call("kdn_short_conv_bwd", _lib.ptr(x), _lib.is_bf16(x), x.stride(0), x.stride(1), _lib.ptr(weight),
                  _lib.is_bf16(weight), _lib.ptr(dy), dy.stride(0) if dy is not None else 0,
                  dy.stride(1) if dy is not None else 0, B, T, D, KERNEL_WIDTH, int(round_preactivation),
                  _lib.ptr(dx), dx.stride(0) if dx is not None else 0, dx.stride(1) if dx is not None else 0,
                  _lib.ptr(dweight), _lib.ptr(ws), ws_bytes, _lib.stream_of(x), tag="short_conv_bwd")


def _check_rows(name, t):
    if t.stride(-1) != 1 or t.stride(1) % 8 or t.stride(0) % 8 or t.data_ptr() % 16:
        raise ValueError(f"{name} needs unit channel stride and 16-byte aligned rows")


# ---------------------------------------------------------------------------
# FLA causal_conv1d (fixed length, per tensor)
# ---------------------------------------------------------------------------

class _ShortConvFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight):
        ctx.save_for_backward(x, weight)
        ctx.set_materialize_grads(False)
        return _conv_fwd(x, weight)

    @staticmethod
    @once_differentiable
    def backward(ctx, dy):
        x, weight = ctx.saved_tensors
        if dy is None:
            return None, None
        dy = dy.to(x.dtype).contiguous()
        dx = torch.empty_like(x) if ctx.needs_input_grad[0] else None
        dw = torch.empty_like(weight) if ctx.needs_input_grad[1] else None
        _conv_bwd(x, weight, dy, dx, dw, round_preactivation=False)
        return dx, dw


def causal_conv1d(x, weight, bias=None, residual=None, initial_state=None, output_final_state=False,
                  activation="silu", backend=None, cu_seqlens=None, chunk_indices=None):
    """Fixed-length causal depthwise convolution + SiLU (FLA ``causal_conv1d`` as called by
    ``lit_gpt/diag_kdn.py:82-95``).  x [B,T,D] bf16/fp32, weight [D,4]; returns ``(y, None)``.
    Only the reference's configuration is accepted: no bias, residual, initial or final state,
    variable lengths; activation "silu"."""
    if bias is not None or residual is not None or initial_state is not None or output_final_state:
        raise NotImplementedError("only the fixed-length, biasless, stateless convolution is supported")
    if cu_seqlens is not None or chunk_indices is not None:
        raise NotImplementedError("variable-length sequences are not supported")
    if activation not in ("silu", "swish"):
        raise NotImplementedError(f"activation {activation!r} is not supported (silu only)")
    if not isinstance(x, torch.Tensor) or x.ndim != 3:
        raise ValueError(f"x must be rank-3 [B,T,D], got {getattr(x, 'shape', None)}")
    B, T, D = x.shape
    if B < 1 or T < 1:
        raise ValueError("batch and sequence dimensions must be positive")
    if weight.shape != (D, KERNEL_WIDTH):
        raise ValueError(f"weight must be [{D},{KERNEL_WIDTH}], got {tuple(weight.shape)}")
    if x.dtype not in (torch.bfloat16, torch.float32) or weight.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("x and weight must be bfloat16 or float32")
    if D % 8:
        raise ValueError("D must be a multiple of 8")
    _lib.require_device(x, weight)
    weight = weight.contiguous()
    if x.stride(-1) != 1:
        x = x.contiguous()
    _check_rows("x", x)
    if torch.is_grad_enabled() and (x.requires_grad or weight.requires_grad):
        return _ShortConvFunction.apply(x, weight), None
    return _conv_fwd(x, weight), None


# ---------------------------------------------------------------------------
# iso packed q|k|v convolution (reference iso_kdn_chunk.py:280-478)
# ---------------------------------------------------------------------------

def _validate_qkv_conv_inputs(x: torch.Tensor, weight: torch.Tensor) -> int:
    """Reference iso_kdn_chunk.py:257-283."""
    if x.ndim != 3:
        raise ValueError(f"packed input must be rank-3 [B,T,3D], got {tuple(x.shape)}")
    if x.shape[0] < 1 or x.shape[1] < 1:
        raise ValueError(f"batch and sequence dimensions must be positive, got {tuple(x.shape)}")
    packed_width = x.shape[-1]
    if packed_width < GROUPS or packed_width % GROUPS != 0:
        raise ValueError(f"packed input width must be a positive multiple of {GROUPS}, got {packed_width}")
    if weight.shape != (packed_width, KERNEL_WIDTH):
        raise ValueError(f"packed weight must be [{packed_width},{KERNEL_WIDTH}], got {tuple(weight.shape)}")
    if not x.is_cuda or weight.device != x.device:
        raise ValueError("QKV causal convolution requires colocated CUDA tensors")
    allowed_dtypes = (torch.bfloat16, torch.float32)
    if x.dtype not in allowed_dtypes:
        raise TypeError(f"packed input must be bfloat16 or float32, got {x.dtype}")
    if weight.dtype not in allowed_dtypes:
        raise TypeError(f"packed weight must be bfloat16 or float32, got {weight.dtype}")
    if not x.is_contiguous() or not weight.is_contiguous():
        raise ValueError("packed input and weight must already be contiguous")
    d = packed_width // GROUPS
    if d % 8:
        raise ValueError("the per-group width must be a multiple of 8")
    return d


def _prepare_gradient(name, gradient, *, B, T, D, device, dtype):
    """Reference iso_kdn_chunk.py:286-311 (None -> zeros; shape, dtype and layout checked)."""
    if gradient is None:
        return None
    expected_shape = (B, T, D)
    if gradient.shape != expected_shape:
        raise ValueError(f"{name} must have shape {expected_shape}, got {tuple(gradient.shape)}")
    if gradient.device != device or gradient.dtype != dtype:
        raise TypeError(f"{name} must be a {dtype} tensor on {device}")
    if not gradient.is_contiguous():
        raise ValueError(f"{name} must already have the standard contiguous layout")
    return gradient


class _QKVCausalConv1d(torch.autograd.Function):
    """Reference iso_kdn_chunk.py:440-465."""

    @staticmethod
    def forward(ctx, x, weight):
        D = _validate_qkv_conv_inputs(x, weight)
        ctx.save_for_backward(x, weight)
        ctx.set_materialize_grads(False)
        return tuple(_conv_fwd(x[..., g * D:(g + 1) * D], weight[g * D:(g + 1) * D]) for g in range(GROUPS))

    @staticmethod
    @once_differentiable
    def backward(ctx, dq, dk, dv):
        if dq is None and dk is None and dv is None:
            return None, None
        x, weight = ctx.saved_tensors
        D = x.shape[-1] // GROUPS
        B, T, _ = x.shape
        grads = [_prepare_gradient(n, g, B=B, T=T, D=D, device=x.device, dtype=x.dtype)
                 for n, g in (("dq", dq), ("dk", dk), ("dv", dv))]
        dx = torch.empty_like(x)
        dw = torch.empty_like(weight)
        for g in range(GROUPS):
            _conv_bwd(x[..., g * D:(g + 1) * D], weight[g * D:(g + 1) * D], grads[g], dx[..., g * D:(g + 1) * D],
                      dw[g * D:(g + 1) * D], round_preactivation=True)
        return dx, dw


def qkv_causal_conv1d(x: torch.Tensor, weight: torch.Tensor):
    """Fixed-length SiLU causal convolution of packed Q/K/V channels (reference
    iso_kdn_chunk.py:468-478).  T = 1 equals the reference's one-token update with a zero cache."""
    d = _validate_qkv_conv_inputs(x, weight)
    if not torch.is_grad_enabled() or not (x.requires_grad or weight.requires_grad):
        return tuple(_conv_fwd(x[..., g * d:(g + 1) * d], weight[g * d:(g + 1) * d]) for g in range(GROUPS))
    return _QKVCausalConv1d.apply(x, weight)


def short_conv_step(x: torch.Tensor, tail: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """One token of the SiLU short convolution from its 3 carried inputs (decoding, no autograd):
    x [B,1,D] (unit channel stride; for B > 1 a batch stride that is a multiple of 8), ``tail`` [B,3,D] contiguous in x's
    dtype, ``weight`` [D,4] contiguous.  Returns y [B,1,D], equal to the convolution of [tail, x]
    at its last token, and advances ``tail`` in place to its last 2 rows and x (``kdn_short_conv_step``)."""
    if x.ndim != 3 or x.shape[1] != 1 or x.stride(-1) != 1:
        raise ValueError(f"x must be [B,1,D] with unit channel stride, got {tuple(x.shape)}")
    B, _, D = x.shape
    if tail.shape != (B, KERNEL_WIDTH - 1, D) or tail.dtype != x.dtype or not tail.is_contiguous():
        raise ValueError(f"tail must be a contiguous {x.dtype} tensor of shape {(B, KERNEL_WIDTH - 1, D)}")
    if weight.shape != (D, KERNEL_WIDTH) or not weight.is_contiguous():
        raise ValueError(f"weight must be a contiguous [{D},{KERNEL_WIDTH}] tensor")
    _lib.require_device(x, tail, weight)
    y = torch.empty((B, 1, D), device=x.device, dtype=x.dtype)
    with torch.cuda.device(x.device):
        _lib.call("kdn_short_conv_step", _lib.ptr(x), _lib.is_bf16(x), x.stride(0), _lib.ptr(tail), tail.stride(0),
                  _lib.ptr(weight), _lib.is_bf16(weight), B, D, _lib.ptr(y), y.stride(0), _lib.stream_of(x))
    return y


__all__ = ("causal_conv1d", "qkv_causal_conv1d", "short_conv_step", "GROUPS", "KERNEL_WIDTH")
