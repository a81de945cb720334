"""The fused isotropic front (``iso_kdn_front``: gate frontend -> scalar gain in one op) against the two
ops it replaces, ``_iso_kdn_gate_precumsum_paired`` -> ``iso_kdn_gain`` (each pinned to the CPU oracle
by its own tests), on the same inputs: g_cumsum, beta, the final precision and every gradient.

The cases reach each path of the fused kernels:

* H = 3, 18: the gain's emit stages the chunk maps in LDS (H <= 26); H = 40: it reads them directly;
* T = 4100: 65 chunks, so the backward's carry composes two groups of 64 chunk maps and the forward's
  lanes read chunk maps past the 64 staged ones;
* T = 1, 64, 130: a single token, one full chunk, a ragged last chunk;
* K = 40 and a misaligned g_raw: the scalar kernels (the two ops one after the other, inside the entry);
* the prior: the gate's mu, a given [H] precision, a given [B,H] precision with the final precision's
  cotangent (state continuation);
* unit (info_scale = K) and non-unit posterior scale; bf16 and fp32 raw inputs.

One case is also compared with the fp64 oracle directly (``ko.iso_gate_frontend`` ->
``ko.iso_gain_unit_key``).  Tolerances: the fused kernels compose the gain's maps in another order
than the separate ones (fp32 rounding), 2e-5 on values and 2e-4 on gradients."""
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


def _inputs(B, T, H, K, dtype, seed, prec):
    g = torch.Generator().manual_seed(seed)
    g_raw = torch.randn(B, T, H, K, generator=g).to(dtype)
    orr_full = torch.randn(B, T, 3 * H, generator=g).to(dtype)
    ob, rb = 0.1 * torch.randn(H, generator=g), 0.1 * torch.randn(H, generator=g)
    A_log = torch.log(torch.empty(H).uniform_(1, 16, generator=g))
    dt = 0.3 * torch.randn(H * K, generator=g)
    mup = torch.randn(H, generator=g)
    init = None
    if prec == "H":
        init = 0.5 + torch.rand(H, generator=g)
    elif prec == "BH":
        init = 0.5 + torch.rand(B, H, generator=g)
    cot = (torch.randn(B, T, H, K, generator=g), torch.randn(B, T, H, generator=g), torch.randn(B, H, generator=g))
    return (g_raw, orr_full, ob, rb, A_log, dt, mup, init), cot


def _leaves(xs, dev, misalign=False):
    out = []
    for i, x in enumerate(xs):
        if x is None:
            out.append(None)
            continue
        if i == 0 and misalign:
            buf = torch.empty(x.numel() + 1, dtype=x.dtype, device=dev)
            y = buf[1:].view(x.shape)
            y.copy_(x.to(dev))
            assert y.data_ptr() % 16 != 0
        else:
            y = x.to(dev)
        out.append(y.requires_grad_(True))
    return out


def _run(fused, leaves, cot, K, info_scale, final):
    from lit_gpt.kdn_ops.iso_kdn_chunk import _iso_kdn_gate_precumsum_paired, iso_kdn_front, iso_kdn_gain
    g_raw, orr_full, ob, rb, A_log, dt, mup, init = leaves
    H = ob.shape[0]
    orr = orr_full[..., H:]
    if fused:
        out = iso_kdn_front(g_raw, orr, ob, rb, A_log, dt, mup, 0.05, 0.01, head_dim=K, info_scale=info_scale,
                            initial_precision=init, output_final_state=final)
    else:
        gc, a, w, r, mu = _iso_kdn_gate_precumsum_paired(g_raw, orr, ob, rb, A_log, dt, mup, 0.05, 0.01)
        gain = iso_kdn_gain(a, w, r, mu if init is None else init, head_dim=K, out_dtype=torch.float32,
                            info_scale=info_scale, output_final_state=final)
        out = (gc, *gain) if final else (gc, gain)
    dev = g_raw.device
    loss = (out[0] * cot[0].to(dev)).sum() + (out[1] * cot[1].to(dev)).sum()
    if final:
        loss = loss + (out[2] * cot[2].to(dev)).sum()
    wrt = [x for x in leaves if x is not None]
    return out, torch.autograd.grad(loss, wrt)


CASES = [
    # B, T, H, K, dtype, info_scale, prec, final, misalign
    (2, 130, 3, 128, torch.bfloat16, None, "mu", False, False),
    (1, 64, 18, 128, torch.bfloat16, None, "mu", True, False),
    (2, 1, 4, 64, torch.float32, 64.0, "mu", False, False),
    (2, 4100, 3, 128, torch.bfloat16, None, "BH", True, False),
    (1, 200, 40, 64, torch.bfloat16, 32.0, "H", True, False),
    (3, 300, 5, 128, torch.float32, None, "BH", True, False),
    (2, 77, 5, 40, torch.bfloat16, None, "mu", True, False),
    (2, 150, 3, 128, torch.bfloat16, None, "BH", True, True),
]


@pytest.mark.parametrize("B,T,H,K,dtype,info_scale,prec,final,misalign", CASES)
def test_iso_front_matches_the_two_ops(B, T, H, K, dtype, info_scale, prec, final, misalign):
    dev = gpu_or_skip()
    log(f"case iso front B={B} T={T} H={H} K={K} {dtype} info_scale={info_scale} prior={prec} final={final} "
        f"misaligned={misalign}")
    xs, cot = _inputs(B, T, H, K, dtype, seed=B * 1000 + T + H, prec=prec)
    # a misaligned g_raw sends both to the scalar gate kernels (bf16 dg_raw rounds alike)
    ref_out, ref_grads = _run(False, _leaves(xs, dev, misalign), cot, K, info_scale, final)
    out, grads = _run(True, _leaves(xs, dev, misalign), cot, K, info_scale, final)
    for name, x, y in zip(("g_cumsum", "beta", "final_precision"), out, ref_out):
        _check(name, x, y, 2e-5)
    names = ["dg_raw", "domega_r_raw", "domega_bias", "dr_bias", "dA_log", "ddt_bias", "dmu_param"]
    if prec != "mu":
        names.append("d_initial_precision")
    for name, x, y in zip(names, grads, ref_grads):
        _check(name, x, y, 2e-4)


def test_iso_front_matches_the_oracle():
    """B2 T130 H3 K128 with a [B,H] prior and the final precision: against the fp64 oracle, tolerances of
    the separate ops' own oracle tests (gate 1e-5 / 1e-2 on the bf16 raw gradients, gain 1e-4)."""
    dev = gpu_or_skip()
    log("case iso front vs oracle B=2 T=130 H=3 K=128 prior [B,H]")
    B, T, H, K = 2, 130, 3, 128
    xs, cot = _inputs(B, T, H, K, torch.bfloat16, seed=7, prec="BH")
    g_raw, orr_full, ob, rb, A_log, dt, mup, init = xs
    ld = [x.double().requires_grad_(True) for x in (g_raw.float(), orr_full[..., H:].float(), ob, rb, A_log, dt, mup,
                                                     init)]
    _gl, gc_, a_, w_, r_, _mu = ko.iso_gate_frontend(*ld[:7], omega_min=0.05, r_min=0.01)
    beta_, c_ = ko.iso_gain_unit_key(a_, w_, r_, ld[7], posterior_scale=1.0, output_final_state=True)
    loss = ((gc_ * math.log(2)) * cot[0].double()).sum() + (beta_ * cot[1].double()).sum() + \
        (c_ * cot[2].double()).sum()
    gref = [torch.zeros_like(x) if gx is None else gx  # mu_param does not reach the outputs with a given prior
            for x, gx in zip(ld, torch.autograd.grad(loss, ld, allow_unused=True))]
    out, grads = _run(True, _leaves(xs, dev), cot, K, None, True)
    _check("g_cumsum", out[0], gc_, 1e-5)
    _check("beta", out[1], beta_, 1e-5)
    _check("final_precision", out[2], c_, 1e-5)
    _check("dg_raw", grads[0], gref[0], 1e-2)
    _check("domega_r_raw", grads[1][..., H:], gref[1], 1e-2)
    for name, x, y in zip(("domega_bias", "dr_bias", "dA_log", "ddt_bias", "dmu_param", "d_initial_precision"),
                          grads[2:], gref[2:]):
        _check(name, x, y, 1e-4)
