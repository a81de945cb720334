"""End-to-end parity of the KDN mixer scan (frontend -> gain -> memory scan, forward and
backward) against the CPU oracle mixers in fp64 with autograd, on identical seeded
inputs with the BASELINE distributions.  Tolerance: max|x-ref|/max|ref| <= 2e-2 for the
bf16 output and every input gradient.  The inputs are bf16, so the oracle
rounds the normalised q, k to bf16 where the production scan does (``round_qk``)."""
import pytest
import torch

from gpu_util import gpu_or_skip, log, rel
from oracle import kdn_oracle as ko

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _run_gpu(variant, inputs, do):
    from lit_gpt.kdn_ops.scan import diag_kdn_scan, iso_kdn_scan
    from lit_gpt.kdn_ops.synthetic import GRAD_KEYS
    leaves = {k: x.clone().requires_grad_(True) for k, x in inputs.items()}
    fn = iso_kdn_scan if variant == "iso" else diag_kdn_scan
    o = fn(**leaves)
    keys = GRAD_KEYS[variant]
    grads = torch.autograd.grad((o.float() * do.float()).sum(), [leaves[k] for k in keys])
    torch.cuda.synchronize()
    return o.float().cpu(), {k: g.float().cpu() for k, g in zip(keys, grads)}


def _run_oracle(variant, inputs, do):
    from lit_gpt.kdn_ops.synthetic import GRAD_KEYS
    leaves = {k: x.detach().cpu().double().requires_grad_(True) for k, x in inputs.items()}
    if variant == "iso":
        o = ko.iso_mixer(**{("q_raw" if k == "q" else "k_raw" if k == "k" else "mu_param"
                             if k == "initial_precision_param" else k): x for k, x in leaves.items()},
                         chunked=True, round_qk=True)
    else:
        o = ko.diag_mixer(**{("q_raw" if k == "q" else "k_raw" if k == "k" else "mu_param"
                              if k == "initial_precision_param" else k): x for k, x in leaves.items()},
                          chunked=True)
    keys = GRAD_KEYS[variant]
    grads = torch.autograd.grad((o * do.cpu().double()).sum(), [leaves[k] for k in keys])
    return o.detach(), dict(zip(keys, grads))


@pytest.mark.parametrize("variant", ["iso", "diag"])
@pytest.mark.parametrize("B,T,H,K", [(2, 200, 2, 64), (1, 130, 2, 128)])
def test_scan_chain_matches_oracle(variant, B, T, H, K):
    dev = gpu_or_skip()
    log(f"case chain {variant} B={B} T={T} H={H} K={K}")
    from lit_gpt.kdn_ops.synthetic import make_inputs
    inputs, do = make_inputs(variant, B, T, H, K, seed=B * 1000 + T, device=dev)
    # non-trivial biases / rates so every parameter gradient is exercised
    g = torch.Generator().manual_seed(T)
    inputs["A_log"] = (0.1 * torch.randn(H, generator=g)).to(dev)
    inputs["initial_precision_param"] = (0.5 * torch.randn(H, generator=g)).to(dev)
    if variant == "iso":
        inputs["omega_bias"] = (0.2 * torch.randn(H, generator=g)).to(dev)
        inputs["r_bias"] = (0.2 * torch.randn(H, generator=g)).to(dev)
    o, grads = _run_gpu(variant, inputs, do)
    o_ref, grads_ref = _run_oracle(variant, inputs, do)
    r = rel(o, o_ref)
    log(f"  o: rel err {r:.3e}")
    assert r < TOL
    for name in grads:
        r = rel(grads[name], grads_ref[name])
        log(f"  d{name}: rel err {r:.3e}")
        assert r < TOL, name
