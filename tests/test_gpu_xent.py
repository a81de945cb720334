"""GPU parity of the fused cross-entropy (kdn_xent_fwd / kdn_xent_bwd) against the CPU oracle.

Losses and log-sum-exps are fp32 outputs of fp32 arithmetic: 1e-5 relative to the larger of 1 and
the largest reference value.  Gradients are written in the logits' dtype: max-relative 1e-5 for
fp32, 2e-2 for bf16 (the north star's bf16 bar), 4e-3 for fp16, the denominator floored at a
tenth of |dloss| * logit_scale (a gradient that is exactly zero in fp64 has no relative scale).
"""
from __future__ import annotations

import pytest
import torch

from gpu_util import gpu_or_skip, log, rel
from oracle import xent_oracle as xo

pytestmark = pytest.mark.gpu

GRAD_TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 4e-3}


def _xent():
    from lit_gpt import fused_cross_entropy as fce
    return fce


def _case(n, C, dtype, seed, dev, ignore_frac=0.2, oob=False, label_dtype=torch.int64):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(n, C, generator=g) * 4).to(dtype)
    y = torch.randint(0, C, (n,), generator=g)
    if n:
        y[torch.rand(n, generator=g) < ignore_frac] = -100
        if oob and n > 2:
            y[1] = C + 7
    return x.to(dev), y.to(label_dtype).to(dev)


def _grad_err(got, ref, d, logit_scale=1.0):
    """max|got - ref| / max(max|ref|, |dloss| logit_scale / 10): the gradient's natural unit is
    |dloss| logit_scale (|p - target| <= 1); the floor keeps a gradient that is exactly zero in
    fp64 (one class with smoothing: p - (1 - s) - s = 0) from dividing rounding by ~1e-17."""
    got = got.detach().double().cpu()
    unit = float(d.detach().abs().max()) * logit_scale / 10 if d.numel() else 0.0
    return float((got - ref).abs().max()) / max(float(ref.abs().max()), unit, 1e-30)


def _loss_err(got, ref):
    return float((got.double().cpu() - ref).abs().max()) / max(1.0, float(ref.abs().max())) if ref.numel() else 0.0


SHAPES = [(1, 1), (7, 33), (64, 32000), (37, 4099), (16, 50304), (0, 128)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,C", SHAPES)
@pytest.mark.parametrize("opts", [dict(), dict(smoothing=0.1), dict(lse_square_scale=1e-4, logit_scale=0.5),
                                  dict(smoothing=0.05, lse_square_scale=2e-3, logit_scale=1.3)])
def test_fwd_bwd_matches_oracle(dtype, n, C, opts):
    dev = gpu_or_skip()
    fce = _xent()
    x, y = _case(n, C, dtype, seed=n * 7 + C, dev=dev, oob=True)
    log(f"xent case n={n} C={C} {dtype} {opts}")
    loss, lse, z = fce.xent_forward(x, y, **opts)
    rl, rlse, rz = xo.xent_forward(x, y, **opts)
    assert _loss_err(loss, rl) <= 1e-5 and _loss_err(lse, rlse) <= 1e-5 and _loss_err(z, rz) <= 1e-5
    d = torch.randn(n, device=dev)
    dx = fce.xent_backward(d, x, lse, y, **opts)
    ref = xo.xent_backward(d, x, rlse, y, **opts)
    if n:
        assert dx.dtype == dtype
        err = _grad_err(dx, ref, d, opts.get("logit_scale", 1.0))
        assert err <= GRAD_TOL[dtype], err


def test_unaligned_rows_and_int32_labels():
    # a row stride that is not a multiple of 16 bytes takes the scalar path
    dev = gpu_or_skip()
    fce = _xent()
    base, y = _case(19, 1001, torch.bfloat16, seed=3, dev=dev, label_dtype=torch.int32)
    x = base[:, 1:]  # row stride 1001 elements, start 2 bytes in
    loss, lse, _ = fce.xent_forward(x, y, smoothing=0.2)
    rl, rlse, _ = xo.xent_forward(x, y, smoothing=0.2)
    assert _loss_err(loss, rl) <= 1e-5 and _loss_err(lse, rlse) <= 1e-5
    d = torch.randn(19, device=dev)
    dx = fce.xent_backward(d, x, lse, y, smoothing=0.2)
    assert rel(dx, xo.xent_backward(d, x, rlse, y, smoothing=0.2)) <= GRAD_TOL[torch.bfloat16]


def test_inplace_backward_and_reductions():
    dev = gpu_or_skip()
    fce = _xent()
    x, y = _case(48, 32000, torch.bfloat16, seed=11, dev=dev)
    for reduction in ("mean", "sum", "none"):
        for zs in (0.0, 1e-4):
            crit = fce.FusedCrossEntropyLoss(reduction=reduction, lse_square_scale=zs, return_z_loss=True)
            a = x.clone().requires_grad_(True)
            loss, zl = crit(a, y)
            rl, rlse, rz = xo.xent_forward(x, y, lse_square_scale=zs)
            keep = float((y != -100).sum())
            red = {"mean": lambda t: t.sum() / keep, "sum": lambda t: t.sum(), "none": lambda t: t}[reduction]
            assert _loss_err(loss.reshape(-1), red(rl).reshape(-1)) <= 1e-5
            assert _loss_err(zl.reshape(-1), red(rz).reshape(-1)) <= 1e-5
            w = torch.randn_like(loss) if reduction == "none" else torch.ones_like(loss)
            loss.backward(w)
            dl = w.double().cpu() * (1.0 / keep if reduction == "mean" else 1.0)
            ref = xo.xent_backward(dl, x, rlse, y, lse_square_scale=zs)
            assert rel(a.grad, ref) <= GRAD_TOL[torch.bfloat16]
            # in-place: the gradient overwrites a copy of the logits and equals the out-of-place one
            b = x.clone()
            b_leaf = b.requires_grad_(True)
            crit_ip = fce.FusedCrossEntropyLoss(reduction=reduction, lse_square_scale=zs, inplace_backward=True)
            crit_ip(b_leaf.view(48, 32000) * 1.0, y).backward(w)  # a non-leaf input is overwritten
            assert torch.equal(b_leaf.grad, a.grad)


def test_three_dim_input_and_precomputed_lse():
    dev = gpu_or_skip()
    fce = _xent()
    x, y = _case(2 * 24, 3000, torch.float32, seed=5, dev=dev)
    crit = fce.FusedCrossEntropyLoss(reduction="none")
    loss3 = crit(x.view(2, 24, 3000), y.view(2, 24))
    loss2 = crit(x, y)
    assert torch.equal(loss3, loss2)
    lse = torch.logsumexp(x.double(), 1).float()
    pre = crit(x, y, precomputed_lse=lse + 0.5)
    keep = y != -100
    assert float((pre[keep] - loss2[keep] - 0.5).abs().max()) <= 1e-5 * max(1.0, float(loss2.abs().max()))
    # a precomputed lse is ignored with label smoothing, as in the reference
    sm = fce.FusedCrossEntropyLoss(reduction="none", label_smoothing=0.1)
    assert torch.equal(sm(x, y, precomputed_lse=lse + 0.5), sm(x, y))


@pytest.mark.parametrize("world", [2, 4])
@pytest.mark.parametrize("zs", [0.0, 1e-3])
def test_vocabulary_split_slices(world, zs):
    # the tensor-parallel mode run slice by slice on one GPU: split-mode losses summed and the
    # slices' lse combined give the whole loss; each slice's backward with the combined lse is
    # the slice of the whole gradient
    dev = gpu_or_skip()
    fce = _xent()
    n, C = 40, 8192
    x, y = _case(n, C, torch.bfloat16, seed=world, dev=dev)
    w = C // world
    losses, lses = [], []
    for r in range(world):
        l, s, z = fce.xent_forward(x[:, r * w:(r + 1) * w].contiguous(), y, smoothing=0.1, lse_square_scale=zs,
                                   total_classes=C, class_start_idx=r * w, split=True)
        assert z is None
        losses.append(l)
        lses.append(s)
    loss, z, lse = fce.finish_split_losses(sum(losses), torch.stack(lses), y, zs, -100)
    rl, rlse, rz = xo.xent_forward(x, y, smoothing=0.1, lse_square_scale=zs)
    assert _loss_err(loss, rl) <= 1e-5 and _loss_err(z, rz) <= 1e-5 and _loss_err(lse, rlse) <= 1e-5
    d = torch.randn(n, device=dev)
    whole = xo.xent_backward(d, x, rlse, y, smoothing=0.1, lse_square_scale=zs)
    for r in range(world):
        part = fce.xent_backward(d, x[:, r * w:(r + 1) * w].contiguous(), lse, y, smoothing=0.1,
                                 lse_square_scale=zs, total_classes=C, class_start_idx=r * w)
        assert rel(part, whole[:, r * w:(r + 1) * w]) <= GRAD_TOL[torch.bfloat16]


def test_rejects_bad_arguments():
    dev = gpu_or_skip()
    fce = _xent()
    x, y = _case(4, 64, torch.float32, seed=0, dev=dev)
    with pytest.raises(TypeError):
        fce.xent_forward(x.double(), y)
    with pytest.raises(TypeError):
        fce.xent_forward(x, y.float())
    with pytest.raises(RuntimeError):  # the C entry rejects a slice outside total_classes
        fce.xent_forward(x, y, total_classes=32)
    with pytest.raises(ValueError):
        fce.FusedCrossEntropyLoss()(x.cpu(), y.cpu())
