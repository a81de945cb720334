"""Fused cross-entropy loss on the HIP kernels ``kdn_xent_fwd`` / ``kdn_xent_bwd``.

Same interface as the reference's ``lit_gpt/fused_cross_entropy.py``: ``CrossEntropyLoss``
(autograd Function, ``:153-294``), ``cross_entropy_loss`` (``:296-334``) and the module
``FusedCrossEntropyLoss`` (``:336-414``) that ``pretrain.py:1165,1258`` applies to the model's
logits.  Per row the kernels compute the log-sum-exp of the scaled logits and the loss with label
smoothing and the optional z-loss (``lse_square_scale * lse**2``); the backward writes the
gradient with respect to the logits, optionally over the logits themselves (``inplace_backward``).

With a ``process_group`` of several ranks each rank holds a slice of the vocabulary (tensor
parallel): the kernel's split mode leaves the log-sum-exp out of each slice's loss, the slices'
log-sum-exps are all-gathered and combined, the losses are summed over the ranks, and the
backward uses the combined log-sum-exp.  There is no CPU path: the tensors must be on the GPU.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from .kdn_ops import _lib

_DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise TypeError(f"logits must be float32, bfloat16 or float16, got {t.dtype}") from None


def _labels_arg(labels: torch.Tensor) -> Tuple[torch.Tensor, int]:
    if labels.dtype == torch.int64:
        return labels.contiguous(), 1
    if labels.dtype == torch.int32:
        return labels.contiguous(), 0
    raise TypeError(f"labels must be int64 or int32, got {labels.dtype}")


def finish_split_losses(losses: torch.Tensor, lse_slices: torch.Tensor, labels: torch.Tensor, lse_square_scale: float,
                        ignore_index: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Combine vocabulary slices: ``losses`` [n] is the sum over slices of the split-mode losses,
    ``lse_slices`` [world, n] the slices' log-sum-exps.  Returns (losses, z_losses, lse) of the
    whole vocabulary (``fused_cross_entropy.py:227-248``)."""
    lse = torch.logsumexp(lse_slices, dim=0)
    ignored = labels == ignore_index
    losses = losses + lse
    if lse_square_scale != 0.0:
        z_losses = (lse_square_scale * lse.square()).masked_fill_(ignored, 0.0)
        losses = losses + z_losses
    else:
        z_losses = torch.zeros_like(losses)
    return losses.masked_fill_(ignored, 0.0), z_losses, lse


def xent_forward(logits, labels, *, smoothing=0.0, logit_scale=1.0, lse_square_scale=0.0, ignore_index=-100,
                 total_classes=None, class_start_idx=0, split=False, precomputed_lse=None):
    """One call of ``kdn_xent_fwd`` on a [n_rows, n_cols] slice: (losses, lse, z_losses or None)."""
    n_rows, n_cols = logits.shape
    total_classes = n_cols if total_classes is None else int(total_classes)
    labels, lab64 = _labels_arg(labels)
    _lib.require_device(logits, labels, precomputed_lse)
    losses = torch.empty(n_rows, dtype=torch.float32, device=logits.device)
    if precomputed_lse is not None:
        lse = precomputed_lse.to(torch.float32).contiguous()
        if lse.shape != (n_rows,):
            raise ValueError(f"precomputed_lse must have shape ({n_rows},), got {tuple(lse.shape)}")
    else:
        lse = torch.empty(n_rows, dtype=torch.float32, device=logits.device)
    z_losses = None if split else torch.empty(n_rows, dtype=torch.float32, device=logits.device)
    if n_rows:
        with torch.cuda.device(logits.device):
            _lib.call("kdn_xent_fwd", _lib.ptr(logits), _dtype_code(logits), logits.stride(0), _lib.ptr(labels), lab64,
                      n_rows, n_cols, float(smoothing), float(logit_scale), float(lse_square_scale), int(ignore_index),
                      total_classes, int(class_start_idx), int(bool(split)), int(precomputed_lse is not None),
                      _lib.ptr(losses), _lib.ptr(lse), _lib.ptr(z_losses), _lib.stream_of(logits))
    return losses, lse, z_losses


def xent_backward(dlosses, logits, lse, labels, *, dlogits=None, smoothing=0.0, logit_scale=1.0, lse_square_scale=0.0,
                  ignore_index=-100, total_classes=None, class_start_idx=0):
    """One call of ``kdn_xent_bwd``: the gradient [n_rows, n_cols] in logits' dtype, written to
    ``dlogits`` when given (which may be ``logits`` itself)."""
    n_rows, n_cols = logits.shape
    total_classes = n_cols if total_classes is None else int(total_classes)
    labels, lab64 = _labels_arg(labels)
    if dlogits is None:
        dlogits = torch.empty_like(logits)
    if dlogits.shape != logits.shape or dlogits.dtype != logits.dtype or dlogits.stride(-1) != 1:
        raise ValueError("dlogits must match logits in shape and dtype, with unit column stride")
    dlosses = dlosses.float()
    lse = lse.float().contiguous()
    _lib.require_device(dlosses, logits, lse, labels, dlogits)
    if n_rows:
        with torch.cuda.device(logits.device):
            _lib.call("kdn_xent_bwd", _lib.ptr(dlogits), dlogits.stride(0), _lib.ptr(dlosses), dlosses.stride(0),
                      _lib.ptr(logits), _dtype_code(logits), logits.stride(0), _lib.ptr(lse), _lib.ptr(labels), lab64,
                      n_rows, n_cols, float(smoothing), float(logit_scale), float(lse_square_scale), int(ignore_index),
                      total_classes, int(class_start_idx), _lib.stream_of(logits))
    return dlogits


class CrossEntropyLoss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, labels, precomputed_lse=None, smoothing=0.0, logit_scale=1.0, lse_square_scale=0.0,
                ignore_index=-100, inplace_backward=False, process_group=None):
        if not logit_scale > 0.0:
            raise ValueError(f"logit_scale must be positive, got {logit_scale}")
        if logits.ndim != 2:
            raise ValueError(f"logits must be [n_rows, n_cols], got {tuple(logits.shape)}")
        n_rows, n_cols = logits.shape
        if labels.shape != (n_rows,):
            raise ValueError(f"labels must have shape ({n_rows},), got {tuple(labels.shape)}")
        world_size = 1 if process_group is None else torch.distributed.get_world_size(process_group)
        rank = 0 if process_group is None else torch.distributed.get_rank(process_group)
        total_classes, class_start_idx = world_size * n_cols, rank * n_cols
        if logits.stride(-1) != 1:
            logits = logits.contiguous()
        # as the reference, a precomputed lse is used only where it is the lse of the plain logits
        use_lse = precomputed_lse if (precomputed_lse is not None and logit_scale == 1.0 and smoothing == 0.0) else None
        split = world_size > 1
        losses, lse, z_losses = xent_forward(logits, labels, smoothing=smoothing, logit_scale=logit_scale,
                                             lse_square_scale=lse_square_scale, ignore_index=ignore_index,
                                             total_classes=total_classes, class_start_idx=class_start_idx,
                                             split=split, precomputed_lse=use_lse)
        if split:
            gathered = torch.empty(world_size, n_rows, dtype=lse.dtype, device=lse.device)
            torch.distributed.all_gather_into_tensor(gathered, lse, group=process_group)
            torch.distributed.all_reduce(losses, op=torch.distributed.ReduceOp.SUM, group=process_group)
            losses, z_losses, lse = finish_split_losses(losses, gathered, labels, lse_square_scale, ignore_index)
        ctx.save_for_backward(logits, lse, labels)
        ctx.mark_non_differentiable(z_losses)
        ctx.smoothing, ctx.logit_scale, ctx.lse_square_scale = smoothing, logit_scale, lse_square_scale
        ctx.ignore_index, ctx.inplace_backward = ignore_index, inplace_backward
        ctx.total_classes, ctx.class_start_idx = total_classes, class_start_idx
        return losses, z_losses

    @staticmethod
    def backward(ctx, grad_losses, grad_z_losses):
        del grad_z_losses  # the z-loss output is for logging; its term is inside the losses
        logits, lse, labels = ctx.saved_tensors
        dlogits = xent_backward(grad_losses, logits, lse, labels, dlogits=logits if ctx.inplace_backward else None,
                                smoothing=ctx.smoothing, logit_scale=ctx.logit_scale,
                                lse_square_scale=ctx.lse_square_scale, ignore_index=ctx.ignore_index,
                                total_classes=ctx.total_classes, class_start_idx=ctx.class_start_idx)
        return dlogits, None, None, None, None, None, None, None, None


def cross_entropy_loss(
    logits: torch.Tensor,
    labels: torch.Tensor,
    precomputed_lse: Optional[torch.Tensor] = None,
    label_smoothing: float = 0.0,
    logit_scale: float = 1.0,
    lse_square_scale: float = 0.0,
    ignore_index=-100,
    inplace_backward: bool = False,
    process_group=None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """logits [n, vocab] (float32, bfloat16 or float16), labels [n] int64 or int32; returns
    (losses [n], z_losses [n]) in float32.  ``label_smoothing``: weight of the uniform target;
    ``logit_scale``: logits are multiplied by it first; ``lse_square_scale``: z-loss weight;
    rows labelled ``ignore_index`` get 0; ``inplace_backward`` writes the gradient over the
    logits; ``process_group``: ranks holding consecutive slices of the vocabulary."""
    return CrossEntropyLoss.apply(logits, labels, precomputed_lse, label_smoothing, logit_scale, lse_square_scale,
                                  ignore_index, inplace_backward, process_group)


class FusedCrossEntropyLoss(nn.Module):
    def __init__(self, ignore_index=-100, reduction="mean", label_smoothing=0.0, logit_scale=1.0,
                 lse_square_scale=0.0, inplace_backward=False, process_group=None, return_z_loss=False):
        super().__init__()
        if reduction not in ("mean", "none", "sum"):
            raise NotImplementedError("Only support reduction = 'mean' or 'none' or 'sum'")
        self.ignore_index = ignore_index
        self.reduction = reduction
        self.label_smoothing = label_smoothing
        self.logit_scale = logit_scale
        self.lse_square_scale = lse_square_scale
        self.inplace_backward = inplace_backward
        self.process_group = process_group
        self.return_z_loss = return_z_loss

    def _reduce(self, x, target):
        if self.reduction == "mean":
            return x.sum() / (target != self.ignore_index).sum()
        if self.reduction == "sum":
            return x.sum()
        return x

    def forward(self, input, target, precomputed_lse=None):
        """input [batch, vocab] or [batch, seq, vocab], target [batch] or [batch, seq]."""
        if not (input.is_cuda and target.is_cuda):
            raise ValueError("FusedCrossEntropyLoss takes GPU tensors only")
        if input.ndim == 3:
            input = input.reshape(-1, input.size(-1))
            target = target.reshape(-1)
        loss, z_loss = cross_entropy_loss(input, target, precomputed_lse=precomputed_lse,
                                          label_smoothing=self.label_smoothing, logit_scale=self.logit_scale,
                                          lse_square_scale=self.lse_square_scale, ignore_index=self.ignore_index,
                                          inplace_backward=self.inplace_backward, process_group=self.process_group)
        loss = self._reduce(loss, target)
        if not self.return_z_loss:
            return loss
        return loss, self._reduce(z_loss, target)


__all__ = ("CrossEntropyLoss", "cross_entropy_loss", "FusedCrossEntropyLoss", "finish_split_losses", "xent_forward",
           "xent_backward")
