"""GPU parity of the gain scans, the frontends and the row normalisations against the
CPU oracle (fp64 autograd) on identical seeded inputs."""
import math

import pytest
import torch
import torch.nn.functional as F

from gpu_util import gpu_or_skip, log, rel, reverse_chunk_sum
from oracle import kdn_oracle as ko

pytestmark = pytest.mark.gpu


def _check(name, got, ref, tol):
    r = rel(got, ref)
    log(f"  {name}: rel err {r:.3e} (tol {tol:g})")
    assert r < tol, f"{name} rel err {r:.3e} > {tol}"


def _iso_gain_oracle(a, omega, r, mu, s):
    """Production iso gain on unit keys (the oracle's golden-pinned tokenwise gain)."""
    return ko.iso_gain_unit_key(a, omega, r, mu, posterior_scale=s)[0]


@pytest.mark.parametrize("T", [1, 63, 300, 4100])
@pytest.mark.parametrize("info_scale", [None, 64.0])
def test_iso_gain(T, info_scale):
    dev = gpu_or_skip()
    log(f"case iso gain T={T} info_scale={info_scale}")
    from lit_gpt.kdn_ops.iso_kdn_chunk import iso_kdn_gain
    B, H, K = 3, 4, 128
    g = torch.Generator().manual_seed(T)
    a = torch.sigmoid(2 + 0.5 * torch.randn(B, T, H, generator=g)) ** 2
    omega = F.softplus(torch.randn(B, T, H, generator=g))
    r = 0.01 + F.softplus(torch.randn(B, T, H, generator=g))
    mu = 0.5 + torch.rand(H, generator=g)
    db = torch.randn(B, T, H, generator=g)
    s = (K if info_scale is None else info_scale) / K
    leaves = [x.double().requires_grad_(True) for x in (a, omega, r, mu)]
    ref = _iso_gain_oracle(*leaves, s)
    gref = torch.autograd.grad((ref * db.double()).sum(), leaves)
    gl = [x.to(dev).requires_grad_(True) for x in (a, omega, r, mu)]
    beta = iso_kdn_gain(*gl, head_dim=K, info_scale=info_scale)
    gg = torch.autograd.grad((beta * db.to(dev)).sum(), gl)
    _check("beta", beta, ref, 1e-5)
    for name, x, y in zip(("da", "domega", "dr", "dmu"), gg, gref):
        _check(name, x, y, 1e-4)


@pytest.mark.parametrize("T,prec", [(1, "H"), (100, "H"), (300, "BHK"), (4097, "H")])
def test_diag_gain(T, prec):
    dev = gpu_or_skip()
    log(f"case diag gain T={T} prec={prec}")
    from lit_gpt.kdn_ops.diag_kdn_chunk import _diag_kdn_gain
    B, H, K = 2, 3, 128
    g = torch.Generator().manual_seed(T + 7)
    k = torch.randn(B, T, H, K, generator=g)
    k = k / k.norm(dim=-1, keepdim=True)
    alpha = torch.sigmoid(2 + 0.5 * torch.randn(B, T, H, K, generator=g))
    omega_raw = torch.randn(B, T, H, K, generator=g).bfloat16()
    r_raw = torch.randn(B, T, H, generator=g).bfloat16()
    omega = F.softplus(omega_raw.float())
    r = 0.01 + F.softplus(r_raw.float())
    mu = (0.5 + torch.rand(H, generator=g)) if prec == "H" else (0.3 + torch.rand(B, H, K, generator=g))
    dkap = torch.randn(B, T, H, K, generator=g)
    dfp = torch.randn(B, H, K, generator=g)
    # oracle in fp64, differentiating through omega = softplus(omega_raw), r = 0.01 + softplus(r_raw)
    kd, ad, ord_, rrd, mud = (x.double().requires_grad_(True) for x in (k, alpha, omega_raw.float(),
                                                                          r_raw.float(), mu))
    kap_ref, fp_ref = ko.diag_gain_tokenwise(kd, ad, F.softplus(ord_), 0.01 + F.softplus(rrd), info_scale=float(K),
                                             initial_precision=mud, output_final_state=True)
    loss = (kap_ref * dkap.double()).sum() + (fp_ref * dfp.double()).sum()
    gref = torch.autograd.grad(loss, (kd, ad, ord_, rrd, mud))
    gl = [x.to(dev).contiguous() for x in (k, alpha, omega, r, mu, omega_raw, r_raw)]
    for i in (0, 1, 4, 5, 6):
        gl[i].requires_grad_(True)
    kap, fprec = _diag_kdn_gain(*gl, output_final_state=True)
    gg = torch.autograd.grad((kap * dkap.to(dev)).sum() + (fprec * dfp.to(dev)).sum(),
                             [gl[0], gl[1], gl[5], gl[6], gl[4]])
    _check("kappa", kap, kap_ref, 1e-5)
    _check("final precision", fprec, fp_ref, 1e-5)
    _check("dk", gg[0], gref[0], 1e-4)
    _check("dalpha", gg[1], gref[1], 1e-4)
    _check("domega_raw", gg[2], gref[2], 1e-2)   # bf16 output
    _check("dr_raw", gg[3], gref[3], 1e-2)       # bf16 output
    _check("dmu", gg[4], gref[4], 1e-4)


@pytest.mark.parametrize("T", [1, 64, 200])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_iso_gate_frontend(T, dtype):
    dev = gpu_or_skip()
    log(f"case iso gate T={T} {dtype}")
    from lit_gpt.kdn_ops.iso_kdn_chunk import _iso_kdn_gate_precumsum_paired
    B, H, K = 2, 3, 128
    g = torch.Generator().manual_seed(T + 3)
    g_raw = torch.randn(B, T, H, K, generator=g).to(dtype)
    orr_full = torch.randn(B, T, 3 * H, generator=g).to(dtype)
    orr = orr_full[..., H:]  # strided view with contiguous last dim, like the layer's split
    ob, rb = 0.1 * torch.randn(H, generator=g), 0.1 * torch.randn(H, generator=g)
    A_log = torch.log(torch.empty(H).uniform_(1, 16, generator=g))
    dt = 0.3 * torch.randn(H * K, generator=g)
    mup = torch.randn(H, generator=g)
    cot = [torch.randn(B, T, H, K, generator=g), torch.randn(B, T, H, generator=g),
           torch.randn(B, T, H, generator=g), torch.randn(B, T, H, generator=g), torch.randn(H, generator=g)]
    # oracle: natural-log gate g; the paired cotangent of g_cumsum is the natural-log
    # cotangent before the reverse chunk sum, i.e. d/dg_cumsum * ln2 ... applied to the prefix
    leaves = [x.double().requires_grad_(True) for x in (g_raw.float(), orr.float(), ob, rb, A_log, dt, mup)]
    gl_, gc_, a_, w_, r_, mu_ = ko.iso_gate_frontend(*[x for x in leaves], omega_min=0.05, r_min=0.01)
    # The consumer returns dL/d(prefix in natural-log units); emulate: loss uses gc*ln2 linearly
    loss = ((gc_ * math.log(2)) * cot[0].double()).sum() + (a_ * cot[1].double()).sum() + \
        (w_ * cot[2].double()).sum() + (r_ * cot[3].double()).sum() + (mu_ * cot[4].double()).sum()
    gref = torch.autograd.grad(loss, leaves)
    gl = [x.to(dev) for x in (g_raw, orr_full, ob, rb, A_log, dt, mup)]
    for x in gl:
        x.requires_grad_(True)
    orr_view = gl[1][..., H:]
    outs = _iso_kdn_gate_precumsum_paired(gl[0], orr_view, gl[2], gl[3], gl[4], gl[5], gl[6], 0.05, 0.01)
    _check("g_cumsum", outs[0], gc_, 1e-5)
    _check("a", outs[1], a_, 1e-5)
    _check("omega", outs[2], w_, 1e-5)
    _check("r", outs[3], r_, 1e-5)
    _check("mu", outs[4], mu_, 1e-6)
    loss = sum((o * c.to(dev)).sum() for o, c in zip(outs, cot))
    gg = torch.autograd.grad(loss, gl)
    tol_raw = 1e-2 if dtype == torch.bfloat16 else 1e-4
    _check("dg_raw", gg[0], gref[0], tol_raw)
    _check("domega_r_raw", gg[1][..., H:], gref[1], tol_raw)
    for name, x, y in zip(("domega_bias", "dr_bias", "dA_log", "ddt_bias", "dmu_param"), gg[2:], gref[2:]):
        _check(name, x, y, 1e-4)


@pytest.mark.parametrize("T", [1, 64, 200])
def test_diag_frontend(T):
    dev = gpu_or_skip()
    log(f"case diag frontend T={T}")
    from lit_gpt.kdn_ops.diag_kdn_chunk import _diag_kdn_frontend_precumsum_paired
    B, H, K = 2, 3, 64
    g = torch.Generator().manual_seed(T + 5)
    f = (2 * torch.randn(B, T, H, K, generator=g)).bfloat16()
    f[0, 0, 0, :4] = 60.0  # alpha far below the 1e-6 clamp on the memory path
    z = torch.randn(B, T, H, K, generator=g).bfloat16()
    y = torch.randn(B, T, H, generator=g).bfloat16()
    A_log = torch.log(torch.empty(H).uniform_(1, 16, generator=g))
    dt = 0.3 * torch.randn(H, K, generator=g)
    mup = torch.randn(H, generator=g)
    dG = torch.randn(B, T, H, K, generator=g)
    dal = torch.randn(B, T, H, K, generator=g)
    dmu = torch.randn(H, generator=g)
    leaves = [x.double().requires_grad_(True) for x in (f.float(), A_log, dt, mup)]
    l_mem, gc_, al_, w_, r_, mu_ = ko.diag_frontend(leaves[0], z.double(), y.double(), leaves[1], leaves[2],
                                                    leaves[3], chunk=64)
    loss = ((gc_ * math.log(2)) * dG.double()).sum() + (al_ * dal.double()).sum() + (mu_ * dmu.double()).sum()
    gref = torch.autograd.grad(loss, leaves)
    gl = [x.to(dev) for x in (f, z, y, A_log, dt, mup)]
    for i in (0, 3, 4, 5):
        gl[i].requires_grad_(True)
    outs = _diag_kdn_frontend_precumsum_paired(*gl)
    _check("g_cumsum", outs[0], gc_, 1e-5)
    _check("alpha", outs[1], al_, 1e-5)
    _check("omega", outs[2], w_, 1e-5)
    _check("r", outs[3], r_, 1e-5)
    _check("mu", outs[4], mu_, 1e-6)
    loss = (outs[0] * dG.to(dev)).sum() + (outs[1] * dal.to(dev)).sum() + (outs[4] * dmu.to(dev)).sum()
    gg = torch.autograd.grad(loss, [gl[0], gl[3], gl[4], gl[5]])
    _check("dretention_raw", gg[0], gref[0], 1e-2)
    _check("dA_log", gg[1], gref[1], 1e-4)
    _check("ddt_bias", gg[2], gref[2], 1e-4)
    _check("dmu_param", gg[3], gref[3], 1e-5)


def test_norms():
    dev = gpu_or_skip()
    log("case norms")
    from lit_gpt.kdn_ops.diag_kdn_chunk import _diag_kdn_normalize
    from lit_gpt.kdn_ops import iso_kdn_chunk as ik
    B, T, H, K = 2, 33, 3, 128
    g = torch.Generator().manual_seed(1)
    q = torch.randn(B, T, H, K, generator=g).bfloat16()
    k = torch.randn(B, T, H, K, generator=g).bfloat16()
    k[0, 0, 0] = 0.0  # zero row: clamp branch
    dqm, dkg, dkm = (torch.randn(B, T, H, K, generator=g) for _ in range(3))
    qd, kd = q.double().requires_grad_(True), k.double().requires_grad_(True)
    qn, kn = ko.diag_normalize(qd), ko.diag_normalize(kd)
    loss = (qn * dqm.double()).sum() + (kn * (dkg + dkm.bfloat16().float()).double()).sum()
    gq, gk = torch.autograd.grad(loss, (qd, kd))
    ql, kl = q.to(dev).requires_grad_(True), k.to(dev).requires_grad_(True)
    qm, kgn, km = _diag_kdn_normalize(ql, kl)
    _check("q_memory", qm, qn, 5e-3)
    _check("k_gain", kgn, kn, 1e-6)
    _check("k_memory", km, kn, 5e-3)
    loss = (qm.float() * dqm.to(dev)).sum() + (kgn * dkg.to(dev)).sum() + (km.float() * dkm.to(dev)).sum()
    dq, dk = torch.autograd.grad(loss, (ql, kl))
    _check("dq_raw", dq, gq, 1e-2)
    _check("dk_raw", dk, gk, 1e-2)
    # FLA-convention l2norm (iso path)
    y, rstd = ik._l2norm_fwd(q.to(dev))
    yd = ko.l2norm_fla(q.double())
    _check("l2norm", y, yd, 5e-3)
    dy = torch.randn(B, T, H, K, generator=g).bfloat16()
    qd2 = q.double().requires_grad_(True)
    gref = torch.autograd.grad((ko.l2norm_fla(qd2) * dy.double()).sum(), qd2)[0]
    dx = ik._l2norm_bwd(q.to(dev), rstd, dy.to(dev))
    _check("l2norm bwd", dx, gref, 1e-2)
