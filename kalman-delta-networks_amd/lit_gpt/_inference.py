"""Inference-time caches for the decode path (no autograd).

A decode step runs one token through every block, so every separate small GEMM and dtype cast
is one more launch.  Projections that read the same input are packed into one weight, and the
small gate parameters' fp32 copies are kept, both cached on the owning module and rebuilt when a
source tensor's storage or version changes (``load_state_dict``, an optimiser step, ``.to()``).
The caches are plain attributes, not buffers, so they never enter a state dict.

Memory cost: a packed weight is a second copy of the packed projections (at iso_kdn_1.3B in bf16,
about 33 MB of input projections and 66 MB of SwiGLU w1|w2 per layer, 1.8 GB over 18 layers).  Packing
is therefore limited to modules in eval mode (``module.training`` False) under no_grad, and
``clear_inference_caches(model)`` drops every cache of a model.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

# at most this many rows (B * T) take the packed projections: the launch-bound decode regime;
# longer inputs keep the separate GEMMs, whose outputs are contiguous
PACK_MAX_ROWS = 64
# at most this many rows with bf16 activations and weights go through the weight-streaming GEMV
GEMV_MAX_ROWS = 8


def use_packed(x: torch.Tensor, module: torch.nn.Module) -> bool:
    """The packed-projection path: no autograd, ``module`` in eval mode, at most PACK_MAX_ROWS rows."""
    return not torch.is_grad_enabled() and not module.training and x.numel() // x.shape[-1] <= PACK_MAX_ROWS


def clear_inference_caches(model: torch.nn.Module) -> None:
    """Drop the packed weights and fp32 parameter copies cached on ``model``'s modules."""
    for m in model.modules():
        m.__dict__.pop("_kdn_inference_cache", None)


def _key(tensors):
    return tuple((t.data_ptr(), t._version, t.dtype, t.device) for t in tensors)


def packed_weight(owner, name: str, tensors, row_multiple: int = 1) -> torch.Tensor:
    """torch.cat(tensors, 0) followed by zero rows up to a multiple of ``row_multiple`` rows (so the
    packed product's rows start on aligned addresses), cached on ``owner`` under ``name``."""
    cache = owner.__dict__.setdefault("_kdn_inference_cache", {})
    key = (_key(tensors), row_multiple)
    hit = cache.get(name)
    if hit is None or hit[0] != key:
        parts = [t.detach() for t in tensors]
        rows = sum(t.shape[0] for t in parts)
        pad = (-rows) % row_multiple
        if pad:
            parts.append(parts[0].new_zeros((pad,) + tuple(parts[0].shape[1:])))
        hit = (key, torch.cat(parts, 0))
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


__all__ = ("PACK_MAX_ROWS", "GEMV_MAX_ROWS", "use_packed", "clear_inference_caches", "packed_weight", "as_f32",
           "linear", "swiglu_gate")
