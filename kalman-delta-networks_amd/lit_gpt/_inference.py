"""Inference-time caches for the decode path (no autograd).

A decode step runs one token through every block, so every separate small GEMM and dtype cast
is one more launch.  Projections that read the same input are packed into one weight, and the
small gate parameters' fp32 copies are kept, both cached on the owning module and rebuilt when a
source tensor's storage or version changes (``load_state_dict``, an optimiser step, ``.to()``).
The caches are plain attributes, not buffers, so they never enter a state dict.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

# at most this many rows (B * T) take the packed projections: the launch-bound decode regime;
# longer inputs keep the separate GEMMs, whose outputs are contiguous
PACK_MAX_ROWS = 64
# at most this many rows with bf16 activations and weights go through the weight-streaming GEMV
GEMV_MAX_ROWS = 8


def use_packed(x: torch.Tensor) -> bool:
    return not torch.is_grad_enabled() and x.numel() // x.shape[-1] <= PACK_MAX_ROWS


def _key(tensors):
    return tuple((t.data_ptr(), t._version, t.dtype, t.device) for t in tensors)


def packed_weight(owner, name: str, tensors) -> torch.Tensor:
    """torch.cat(tensors, 0), cached on ``owner`` under ``name``."""
    cache = owner.__dict__.setdefault("_kdn_inference_cache", {})
    key = _key(tensors)
    hit = cache.get(name)
    if hit is None or hit[0] != key:
        hit = (key, torch.cat([t.detach() for t in tensors], 0))
        cache[name] = hit
    return hit[1]


def as_f32(owner, name: str, t: torch.Tensor) -> torch.Tensor:
    """``t.float()``; under no_grad the converted copy of a non-fp32 tensor is cached on ``owner``."""
    if t.dtype == torch.float32 or torch.is_grad_enabled():
        return t.float()
    cache = owner.__dict__.setdefault("_kdn_inference_cache", {})
    key = _key((t,))
    hit = cache.get(name)
    if hit is None or hit[0] != key:
        hit = (key, t.detach().float())
        cache[name] = hit
    return hit[1]


def _gemv_ok(x, weight, bias) -> bool:
    return (not torch.is_grad_enabled() and x.is_cuda and x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
            and (bias is None or bias.dtype == torch.bfloat16) and x.shape[-1] % 8 == 0 and weight.is_contiguous()
            and x.numel() // max(x.shape[-1], 1) <= GEMV_MAX_ROWS
            and not torch.is_autocast_enabled("cuda"))


def linear(x: torch.Tensor, weight: torch.Tensor, bias=None) -> torch.Tensor:
    """``F.linear``; a no-grad call of at most ``GEMV_MAX_ROWS`` rows with bf16 activations, weight
    and bias (the one-token decode step of a bf16 model) reads the weight through ``kdn_gemv``
    instead of a small-M GEMM."""
    if _gemv_ok(x, weight, bias):
        from .kdn_ops.step import kdn_gemv
        return kdn_gemv(x, weight, bias)
    return F.linear(x, weight, bias)


def swiglu_gate(x: torch.Tensor, w12: torch.Tensor) -> torch.Tensor:
    """silu(x w1^T) * (x w2^T) for a packed ``w12`` = [w1; w2]; in the decode regime of ``linear``
    one ``kdn_gemv`` launch computes both products and the gate."""
    if _gemv_ok(x, w12, None) and w12.shape[0] % 2 == 0:
        from .kdn_ops.step import kdn_gemv
        return kdn_gemv(x, w12, None, gated=True)
    h1, h2 = linear(x, w12).chunk(2, dim=-1)
    return F.silu(h1) * h2


__all__ = ("PACK_MAX_ROWS", "GEMV_MAX_ROWS", "use_packed", "packed_weight", "as_f32", "linear", "swiglu_gate")
