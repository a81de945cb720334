"""CPU restatement of the fused cross-entropy loss (TEST INFRASTRUCTURE ONLY).

The parity checker for ``kdn_xent_fwd`` / ``kdn_xent_bwd`` and ``lit_gpt.fused_cross_entropy``.
Only ``tests/`` may import it; the product path never does.  Plain PyTorch on the CPU in fp64.

What each function restates (reference = ngocbh/kalman-delta-networks):

* ``xent_forward``  -- lit_gpt/fused_cross_entropy.py:29-100 (per-row log-sum-exp of the
  scaled logits, label smoothing over ``total_classes``, z-loss, ``ignore_index``, labels
  outside the slice, the vocabulary-split mode that leaves the log-sum-exp and z-loss out)
* ``xent_backward`` -- fused_cross_entropy.py:103-150 (softmax minus the smoothed one-hot,
  the z-loss factor 1 + 2 z lse, scaled by dloss * logit_scale)
* ``combine_split`` -- fused_cross_entropy.py:227-248 (slices' losses summed, log-sum-exps
  combined, then the z-loss and the ignore mask)

Pinned (tests/test_oracle_xent.py) against ``torch.nn.functional.cross_entropy`` with
``label_smoothing`` and ``ignore_index``, against ``torch.logsumexp`` for the z-loss, against
autograd of that library expression for the backward, against an identity of
``F.cross_entropy`` for labels outside the vocabulary, and by splitting the vocabulary into
slices whose combination must equal the whole.
"""
from __future__ import annotations

import torch


def xent_forward(logits, labels, *, smoothing=0.0, logit_scale=1.0, lse_square_scale=0.0, ignore_index=-100,
                 total_classes=None, class_start_idx=0, split=False, precomputed_lse=None):
    """(losses, lse, z_losses) [n] fp64 for logits [n, C] (this slice's C classes)."""
    x = logits.detach().double().cpu() * logit_scale
    n, C = x.shape
    total = C if total_classes is None else int(total_classes)
    lab = labels.detach().cpu().long()
    lse = torch.logsumexp(x, 1) if precomputed_lse is None else precomputed_lse.detach().double().cpu()
    sx = x.sum(1)
    ignored = lab == ignore_index
    li = lab - class_start_idx
    inside = (li >= 0) & (li < C) & ~ignored
    xl = torch.zeros(n, dtype=torch.float64)
    rows = inside.nonzero().flatten()
    xl[rows] = x[rows, li[rows]]
    lse_part = torch.zeros_like(lse) if split else lse
    if smoothing > 0:
        loss = torch.where(inside, lse_part - smoothing * sx / total - (1 - smoothing) * xl,
                           smoothing * (lse_part - sx / total))
    else:
        loss = torch.where(inside, lse_part - xl, torch.zeros_like(lse))
    z = torch.zeros_like(lse) if split else lse_square_scale * lse * lse
    loss = (loss + z).masked_fill(ignored, 0.0)
    z = z.masked_fill(ignored, 0.0)
    return loss, lse, z


def xent_backward(dlosses, logits, lse, labels, *, smoothing=0.0, logit_scale=1.0, lse_square_scale=0.0,
                  ignore_index=-100, total_classes=None, class_start_idx=0):
    """dlogits [n, C] fp64."""
    x = logits.detach().double().cpu() * logit_scale
    n, C = x.shape
    total = C if total_classes is None else int(total_classes)
    lab = labels.detach().cpu().long()
    lse = lse.detach().double().cpu()
    d = dlosses.detach().double().cpu().expand(n).clone()
    d[lab == ignore_index] = 0.0
    p = torch.exp(x - lse[:, None]) * (1 + 2 * lse_square_scale * lse)[:, None]
    li = lab - class_start_idx
    cols = torch.arange(C)[None, :]
    p = p - (1 - smoothing) * (cols == li[:, None]).double() - smoothing / total
    return (d * logit_scale)[:, None] * p


def combine_split(loss_slices, lse_slices, labels, *, lse_square_scale=0.0, ignore_index=-100):
    """Whole-vocabulary (losses, z_losses, lse) from split-mode slices."""
    lse = torch.logsumexp(torch.stack([l.double() for l in lse_slices]), 0)
    loss = sum(l.double() for l in loss_slices) + lse
    ignored = labels.detach().cpu().long() == ignore_index
    z = (lse_square_scale * lse * lse).masked_fill(ignored, 0.0)
    return (loss + z).masked_fill(ignored, 0.0), z, lse


__all__ = ("xent_forward", "xent_backward", "combine_split")
