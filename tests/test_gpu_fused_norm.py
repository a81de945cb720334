"""The isotropic scan's in-op L2 norm folded into the memory scan: the forward normalises the raw
q, k rows as it loads them and writes their rstd (kdn_mem_fwd with q_rstd / k_rstd), the backward
forms the normalised operands again and applies the norm's backward in its kernel (kdn_mem_bwd with
q_rstd / k_rstd); reference iso_kdn_chunk.py:2190-2238, which normalises q and k inside the op
(FLA l2norm_fwd) and applies FLA's l2norm_bwd to dq, dk.

* The forward's rstd and o are bit-identical to kdn_l2norm_fwd followed by the scan on its output.

* Against the unfused composition on the same inputs -- kdn_l2norm_fwd, the scan backward on the
  normalised q, k, kdn_l2norm_bwd -- which the other memory-scan tests pin to the fp64 oracle: dv,
  dbeta, dg and the initial-state gradient are bit-identical (both take the same normalised operands),
  and dq, dk agree to 1e-2 (the composition rounds the normalised gradient to bf16 and recomputes
  y = x rstd in fp32; the fused kernel keeps the gradient in fp32 and takes y as the bf16 operand).
* Against the fp64 oracle with the norm inside the autograd graph (oracle.l2norm_fla, the normalised
  q, k rounded to bf16 as the forward does, straight-through): dq, dk at the bf16-output tolerance.
Shapes: K = V = 128 with a ragged last chunk and one chunk whose decay span sends it to the exact
per-block path (its dq, dk get the norm's backward from a separate pass over the flagged rows), and
K = V = 64 (half the kernel's waves own no channel tile).
"""
import pytest
import torch

from gpu_util import chunk_prefix_base2, gpu_or_skip, log, rel
from oracle import kdn_oracle as ko

pytestmark = pytest.mark.gpu
CHUNK = 64


def _inputs(seed, B, T, H, K, V, extreme_chunk):
    g = torch.Generator().manual_seed(seed)
    q = (1.7 * torch.randn(B, T, H, K, generator=g)).bfloat16()   # raw, not unit norm
    k = (0.6 * torch.randn(B, T, H, K, generator=g)).bfloat16()
    v = torch.randn(B, T, H, V, generator=g).bfloat16()
    ell = (-0.13 + 0.05 * torch.randn(B, T, H, K, generator=g)).clamp(max=0.0)
    if extreme_chunk:
        ell[:, 64:128] = (-8.0 + 2.0 * torch.randn(B, 64, H, K, generator=g)).clamp(max=0.0)
    beta = 0.2 + 0.8 * torch.rand(B, T, H, generator=g)
    do = torch.randn(B, T, H, V, generator=g).bfloat16()
    h0 = 0.3 * torch.randn(B, H, K, V, generator=g)
    return q, k, v, ell, beta, do, h0


@pytest.mark.parametrize("B,T,H,K,V,extreme", [(2, 200, 2, 128, 128, True), (1, 130, 2, 64, 64, False)])
def test_fused_norm_backward_matches_composition_and_oracle(B, T, H, K, V, extreme):
    dev = gpu_or_skip()
    from lit_gpt.kdn_ops import iso_kdn_chunk as ik
    log(f"case fused-norm iso B={B} T={T} H={H} K={K} V={V} extreme_chunk={extreme}")
    q, k, v, ell, beta, do, h0 = _inputs(7 + T + K, B, T, H, K, V, extreme)
    scale = K ** -0.5
    G2 = chunk_prefix_base2(ell, CHUNK).float()
    qg, kg, vg, Gg, bg, dog, h0g = (x.to(dev).contiguous() for x in (q, k, v, G2, beta.float(), do, h0.float()))

    # the op with the norm inside (fused backward)
    leaves = [x.clone().requires_grad_(True) for x in (qg, kg, vg, Gg, bg, h0g)]
    o = ik._chunk_kda_precumsum_paired(leaves[0], leaves[1], leaves[2], leaves[3], leaves[4], scale,
                                       initial_state=leaves[5])
    fused = torch.autograd.grad(o, leaves, grad_outputs=dog)
    # the unfused composition
    qn, q_rstd = ik._l2norm_fwd(qg)
    kn, k_rstd = ik._l2norm_fwd(kg)
    o2, saved, _ = ik._chunk_kda_fwd_precum(qn, kn, vg, Gg, bg, scale, initial_state=h0g)
    dqn, dkn, dv, db, dg, dh0 = ik._chunk_kda_bwd_precum(qn, kn, vg, Gg, bg, saved, scale, dog,
                                                         need_initial_state_grad=True)
    dq = ik._l2norm_bwd(qg, q_rstd, dqn)
    dk = ik._l2norm_bwd(kg, k_rstd, dkn)
    # the norm inside the scan forward writes the same rstd as kdn_l2norm_fwd (same sum order)
    q_rs2 = torch.empty_like(q_rstd)
    k_rs2 = torch.empty_like(k_rstd)
    o3, _, _ = ik._chunk_kda_fwd_precum(qg, kg, vg, Gg, bg, scale, initial_state=h0g, q_rstd=q_rs2, k_rstd=k_rs2)
    torch.cuda.synchronize()
    assert torch.equal(q_rs2, q_rstd) and torch.equal(k_rs2, k_rstd), "rstd differs from kdn_l2norm_fwd's"
    assert torch.equal(o3, o2)
    assert torch.equal(o, o2)
    for name, a, b_ in (("dv", fused[2], dv), ("dbeta", fused[4], db), ("d initial state", fused[5], dh0)):
        assert torch.equal(a, b_), f"{name} differs from the unfused composition"
    # the gate cotangent: the op returns it in natural-log coordinates, as the composition does
    assert torch.equal(fused[3], dg), "dg differs from the unfused composition"
    for name, a, b_ in (("dq", fused[0], dq), ("dk", fused[1], dk)):
        r = rel(a.float(), b_.float())
        log(f"  {name} fused vs composition: rel err {r:.3e}")
        assert r <= 1e-2, name

    # fp64 oracle with the norm in the graph
    qd = q.double().requires_grad_(True)
    kd = k.double().requires_grad_(True)
    qnd = ko.amp_round(ko.l2norm_fla(qd), True)
    knd = ko.amp_round(ko.l2norm_fla(kd), True)
    od, _ = ko.memory_tokenwise(qnd, knd, v.double(), ell.double().exp(), beta.double()[..., None] * knd,
                                scale=scale, initial_state=h0.double())
    gq, gk = torch.autograd.grad((od * do.double()).sum(), [qd, kd])
    for name, a, ref in (("dq", fused[0], gq), ("dk", fused[1], gk)):
        r = rel(a.float().cpu(), ref)
        log(f"  {name} vs oracle: rel err {r:.3e}")
        assert r <= 1e-2, name
