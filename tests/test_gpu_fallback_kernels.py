"""GPU parity of the frontends' scalar kernels against the CPU oracle (fp64 autograd).

The gate, retention-frontend and row-norm entry points run vectorised kernels (8 channels per
lane, 16-byte loads) when K is a multiple of 8 that tiles the workgroup and every row pointer is
16-byte aligned; otherwise they run one-channel-per-thread kernels.  These cases reach the latter:

* K = 40 (a multiple of 8 whose 5 channel groups do not tile 256 threads) and K = 36 (not a
  multiple of 8), for the isotropic gate and the FLA-convention L2 norm (the diagonal ops accept
  K in {64, 128} only, as in the reference);
* K = 64 or 128 with the input one element past an aligned address (a contiguous tensor that
  starts inside its storage), which the vector kernels cannot load with 16-byte accesses.

The oracle calls and tolerances are the ones of the vectorised kernels' tests."""
import math

import pytest
import torch

from gpu_util import gpu_or_skip, log, rel
from oracle import kdn_oracle as ko

pytestmark = pytest.mark.gpu


def _check(name, got, ref, tol):
    r = rel(got, ref)
    log(f"  {name}: rel err {r:.3e} (tol {tol:g})")
    assert r < tol, f"{name} rel err {r:.3e} > {tol}"


def _to_dev(x, dev, misalign):
    """``x`` on the GPU; with ``misalign`` the tensor starts one element into a fresh buffer, so its
    data pointer is not 16-byte aligned (it stays contiguous, so no wrapper copies it)."""
    if not misalign:
        return x.to(dev)
    buf = torch.empty(x.numel() + 1, dtype=x.dtype, device=dev)
    y = buf[1:].view(x.shape)
    y.copy_(x.to(dev))
    assert y.is_contiguous() and y.data_ptr() % 16 != 0
    return y


@pytest.mark.parametrize("K,misalign", [(40, False), (36, False), (128, True)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_iso_gate_scalar_kernels(K, misalign, dtype):
    dev = gpu_or_skip()
    log(f"case iso gate scalar kernels K={K} misaligned={misalign} {dtype}")
    from lit_gpt.kdn_ops.iso_kdn_chunk import _iso_kdn_gate_precumsum_paired
    B, T, H = 2, 130, 3
    g = torch.Generator().manual_seed(K + 11)
    g_raw = torch.randn(B, T, H, K, generator=g).to(dtype)
    orr_full = torch.randn(B, T, 3 * H, generator=g).to(dtype)
    orr = orr_full[..., H:]
    ob, rb = 0.1 * torch.randn(H, generator=g), 0.1 * torch.randn(H, generator=g)
    A_log = torch.log(torch.empty(H).uniform_(1, 16, generator=g))
    dt = 0.3 * torch.randn(H * K, generator=g)
    mup = torch.randn(H, generator=g)
    cot = [torch.randn(B, T, H, K, generator=g), torch.randn(B, T, H, generator=g),
           torch.randn(B, T, H, generator=g), torch.randn(B, T, H, generator=g), torch.randn(H, generator=g)]
    leaves = [x.double().requires_grad_(True) for x in (g_raw.float(), orr.float(), ob, rb, A_log, dt, mup)]
    _gl, gc_, a_, w_, r_, mu_ = ko.iso_gate_frontend(*leaves, omega_min=0.05, r_min=0.01)
    loss = ((gc_ * math.log(2)) * cot[0].double()).sum() + (a_ * cot[1].double()).sum() + \
        (w_ * cot[2].double()).sum() + (r_ * cot[3].double()).sum() + (mu_ * cot[4].double()).sum()
    gref = torch.autograd.grad(loss, leaves)
    gl = [_to_dev(g_raw, dev, misalign)] + [x.to(dev) for x in (orr_full, ob, rb, A_log, dt, mup)]
    for x in gl:
        x.requires_grad_(True)
    outs = _iso_kdn_gate_precumsum_paired(gl[0], gl[1][..., H:], gl[2], gl[3], gl[4], gl[5], gl[6], 0.05, 0.01)
    _check("g_cumsum", outs[0], gc_, 1e-5)
    _check("a", outs[1], a_, 1e-5)
    _check("omega", outs[2], w_, 1e-5)
    _check("r", outs[3], r_, 1e-5)
    loss = sum((o * c.to(dev)).sum() for o, c in zip(outs, cot))
    gg = torch.autograd.grad(loss, gl)
    tol_raw = 1e-2 if dtype == torch.bfloat16 else 1e-4
    _check("dg_raw", gg[0], gref[0], tol_raw)
    _check("domega_r_raw", gg[1][..., H:], gref[1], tol_raw)
    for name, x, y in zip(("domega_bias", "dr_bias", "dA_log", "ddt_bias", "dmu_param"), gg[2:], gref[2:]):
        _check(name, x, y, 1e-4)


@pytest.mark.parametrize("K,misalign", [(64, True), (128, True)])
def test_diag_frontend_scalar_kernels(K, misalign):
    dev = gpu_or_skip()
    log(f"case diag frontend scalar kernels K={K} misaligned={misalign}")
    from lit_gpt.kdn_ops.diag_kdn_chunk import _diag_kdn_frontend_precumsum_paired
    B, T, H = 2, 100, 3
    g = torch.Generator().manual_seed(K + 17)
    f = (2 * torch.randn(B, T, H, K, generator=g)).bfloat16()
    f[0, 0, 0, :4] = 60.0  # alpha below the 1e-6 clamp of the memory path
    z = torch.randn(B, T, H, K, generator=g).bfloat16()
    y = torch.randn(B, T, H, generator=g).bfloat16()
    A_log = torch.log(torch.empty(H).uniform_(1, 16, generator=g))
    dt = 0.3 * torch.randn(H, K, generator=g)
    mup = torch.randn(H, generator=g)
    dG = torch.randn(B, T, H, K, generator=g)
    dal = torch.randn(B, T, H, K, generator=g)
    dmu = torch.randn(H, generator=g)
    leaves = [x.double().requires_grad_(True) for x in (f.float(), A_log, dt, mup)]
    _l, gc_, al_, w_, r_, mu_ = ko.diag_frontend(leaves[0], z.double(), y.double(), leaves[1], leaves[2],
                                                 leaves[3], chunk=64)
    loss = ((gc_ * math.log(2)) * dG.double()).sum() + (al_ * dal.double()).sum() + (mu_ * dmu.double()).sum()
    gref = torch.autograd.grad(loss, leaves)
    gl = [_to_dev(f, dev, misalign)] + [x.to(dev) for x in (z, y, A_log, dt, mup)]
    for i in (0, 3, 4, 5):
        gl[i].requires_grad_(True)
    outs = _diag_kdn_frontend_precumsum_paired(*gl)
    _check("g_cumsum", outs[0], gc_, 1e-5)
    _check("alpha", outs[1], al_, 1e-5)
    _check("omega", outs[2], w_, 1e-5)
    _check("r", outs[3], r_, 1e-5)
    loss = (outs[0] * dG.to(dev)).sum() + (outs[1] * dal.to(dev)).sum() + (outs[4] * dmu.to(dev)).sum()
    gg = torch.autograd.grad(loss, [gl[0], gl[3], gl[4], gl[5]])
    _check("dretention_raw", gg[0], gref[0], 1e-2)
    _check("dA_log", gg[1], gref[1], 1e-4)
    _check("ddt_bias", gg[2], gref[2], 1e-4)
    _check("dmu_param", gg[3], gref[3], 1e-5)


@pytest.mark.parametrize("K,misalign", [(36, False), (40, False), (64, True), (128, True)])
def test_row_norm_scalar_kernels(K, misalign):
    dev = gpu_or_skip()
    log(f"case row norms scalar kernels K={K} misaligned={misalign}")
    from lit_gpt.kdn_ops import iso_kdn_chunk as ik
    from lit_gpt.kdn_ops.diag_kdn_chunk import _diag_kdn_normalize
    B, T, H = 2, 33, 3
    g = torch.Generator().manual_seed(K + 23)
    q = torch.randn(B, T, H, K, generator=g).bfloat16()
    k = torch.randn(B, T, H, K, generator=g).bfloat16()
    k[0, 0, 0] = 0.0  # zero row: the clamp branch
    dqm, dkg, dkm = (torch.randn(B, T, H, K, generator=g) for _ in range(3))
    dy = torch.randn(B, T, H, K, generator=g).bfloat16()
    # FLA-convention l2norm (the isotropic path's separate norm)
    qx = _to_dev(q, dev, misalign)
    y, rstd = ik._l2norm_fwd(qx)
    _check("l2norm", y, ko.l2norm_fla(q.double()), 5e-3)
    qd2 = q.double().requires_grad_(True)
    gref = torch.autograd.grad((ko.l2norm_fla(qd2) * dy.double()).sum(), qd2)[0]
    dx = ik._l2norm_bwd(qx, rstd, _to_dev(dy, dev, misalign))
    _check("l2norm bwd", dx, gref, 1e-2)
    if K not in (64, 128):
        return
    qd, kd = q.double().requires_grad_(True), k.double().requires_grad_(True)
    qn, kn = ko.diag_normalize(qd), ko.diag_normalize(kd)
    loss = (qn * dqm.double()).sum() + (kn * (dkg + dkm.bfloat16().float()).double()).sum()
    gq, gk = torch.autograd.grad(loss, (qd, kd))
    ql, kl = _to_dev(q, dev, misalign).requires_grad_(True), _to_dev(k, dev, misalign).requires_grad_(True)
    qm, kgn, km = _diag_kdn_normalize(ql, kl)
    _check("q_memory", qm, qn, 5e-3)
    _check("k_gain", kgn, kn, 1e-6)
    _check("k_memory", km, kn, 5e-3)
    loss = (qm.float() * dqm.to(dev)).sum() + (kgn * dkg.to(dev)).sum() + (km.float() * dkm.to(dev)).sum()
    dq, dk = torch.autograd.grad(loss, (ql, kl))
    _check("dq_raw", dq, gq, 1e-2)
    _check("dk_raw", dk, gk, 1e-2)
