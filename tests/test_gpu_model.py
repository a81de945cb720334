"""GPU parity of the config-4 block stack against the CPU oracle composition.

* ``FusedRMSNorm`` (kdn_rms_norm_* through the C ABI): y, dx, dweight at 1e-5 (fp32) / 2e-2
  (bf16), at the model width 2304 and a narrow width, plus bit-identical repeated weight
  gradients (fixed-order sums).
* Isotropic layer in fp32 eval mode against the fp64 oracle layer (``ko.iso_layer``): output and
  every parameter / input gradient at 2e-2 (the scan stores q, k, v in bf16 on this path, as the
  reference's does).
* Isotropic and diagonal layers in training mode under CUDA bf16 autocast (the reference's only
  training configuration) against the oracle with autocast's bf16 rounding points (``amp=True``):
  output and gradients at 2e-2.
* A two-layer isotropic GPT in fp32 eval mode against the fp64 oracle GPT at 2e-2, and a
  two-layer GPT of each mixer under autocast against the autocast oracle, each quantity at
  2e-2 (the oracle rounds bf16 cotangents as autograd does): logits and the gradients of the embedding,
  the first block's norms / mixer input projection, a mixer's A_log, the final norm and the head.
"""
import pytest
import torch

from gpu_util import gpu_or_skip, log, rel
from oracle import kdn_oracle as ko

pytestmark = pytest.mark.gpu
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}
TOL_LAYER = 2e-2


def _check(name, got, ref, tol):
    r = rel(got, ref)
    log(f"  {name}: rel err {r:.3e} (tol {tol:g})")
    assert r <= tol, f"{name}: {r:.3e} > {tol}"


@pytest.mark.parametrize("rows,D,dtype", [(300, 2304, torch.bfloat16), (300, 2304, torch.float32),
                                          (1, 128, torch.float32), (4096, 128, torch.bfloat16),
                                          (7, 8192, torch.bfloat16)])
def test_rms_norm_matches_oracle(rows, D, dtype):
    dev = gpu_or_skip()
    from lit_gpt.rmsnorm import FusedRMSNorm
    log(f"case rms norm rows={rows} D={D} {dtype}")
    g = torch.Generator().manual_seed(rows + D)
    x = (3.0 * torch.randn(rows, D, generator=g)).to(dtype)
    w = 1.0 + 0.1 * torch.randn(D, generator=g)
    dy = torch.randn(rows, D, generator=g).to(dtype)
    xd, wd = x.double().requires_grad_(True), w.double().requires_grad_(True)
    y_ref = ko.rms_norm(xd, wd, 1e-5)
    dx_ref, dw_ref = torch.autograd.grad((y_ref * dy.double()).sum(), (xd, wd))
    norm = FusedRMSNorm(D, eps=1e-5).to(dev)
    with torch.no_grad():
        norm.weight.copy_(w)
    xg = x.to(dev).requires_grad_(True)
    y = norm(xg)
    assert y.dtype == dtype
    dx, dw = torch.autograd.grad(y, (xg, norm.weight), dy.to(dev))
    dw2 = torch.autograd.grad(norm(xg), norm.weight, dy.to(dev))[0]
    torch.cuda.synchronize()
    tol = TOL[dtype]
    _check("y", y, y_ref, tol)
    _check("dx", dx, dx_ref, tol)
    _check("dweight", dw, dw_ref, tol)
    assert torch.equal(dw, dw2)


def _layer(variant, dev, seed, head_dim=64):
    torch.manual_seed(seed)
    if variant == "iso":
        from lit_gpt.iso_kdn import IsotropicKalmanDeltaNetwork as L
    else:
        from lit_gpt.diag_kdn import DiagonalKalmanDeltaNetwork as L
    layer = L(hidden_size=2 * head_dim, head_dim=head_dim, num_heads=2)
    with torch.no_grad():
        # move off the zero / one initial values so every parameter's gradient is exercised
        for name, p in layer.named_parameters():
            if "omega_proj.1" in name or "o_norm" in name:
                p.add_(0.05 * torch.randn_like(p))
    return layer.to(dev)


def _oracle_params(layer):
    return {k: v.detach().cpu().double().requires_grad_(True) for k, v in layer.state_dict().items()}


def _compare_layer(layer, p_ref, x, xg, out, out_ref, dy):
    _check("output", out, out_ref, TOL_LAYER)
    names = list(p_ref)
    grads_ref = torch.autograd.grad((out_ref * dy.double()).sum(), [x] + [p_ref[n] for n in names],
                                    allow_unused=True)
    params = dict(layer.named_parameters())
    grads = torch.autograd.grad(out, [xg] + [params[n] for n in names], dy.to(out.device).to(out.dtype),
                                allow_unused=True)
    torch.cuda.synchronize()
    _check("d hidden", grads[0], grads_ref[0], TOL_LAYER)
    for n, gg, gr in zip(names, grads[1:], grads_ref[1:]):
        assert gg is not None and gr is not None, n
        _check(f"d {n}", gg, gr, TOL_LAYER)


def test_iso_layer_fp32_eval_matches_oracle():
    dev = gpu_or_skip()
    B, T = 2, 130
    log(f"case iso layer fp32 eval B={B} T={T} H=2 K=64")
    layer = _layer("iso", dev, 0).eval()
    g = torch.Generator().manual_seed(11)
    x = torch.randn(B, T, 128, generator=g)
    dy = torch.randn(B, T, 128, generator=g).bfloat16().float()  # exact in bf16 and fp32
    p_ref = _oracle_params(layer)
    xd = x.double().requires_grad_(True)
    out_ref = ko.iso_layer(p_ref, xd, info_scale=64.0)
    xg = x.to(dev).requires_grad_(True)
    out, _, _ = layer(xg)
    assert out.dtype == torch.float32
    _compare_layer(layer, p_ref, xd, xg, out, out_ref, dy)


@pytest.mark.parametrize("variant,head_dim", [("iso", 64), ("diag", 64), ("iso", 128), ("diag", 128)])
def test_layer_bf16_autocast_training_matches_oracle(variant, head_dim):
    dev = gpu_or_skip()
    B, T, D = 2, 130, 2 * head_dim
    log(f"case {variant} layer autocast training B={B} T={T} H=2 K={head_dim}")
    layer = _layer(variant, dev, 1, head_dim).train()
    g = torch.Generator().manual_seed(12)
    x = torch.randn(B, T, D, generator=g)
    dy = torch.randn(B, T, D, generator=g).bfloat16().float()  # exact in bf16 and fp32
    p_ref = _oracle_params(layer)
    xd = x.double().requires_grad_(True)
    if variant == "iso":
        out_ref = ko.iso_layer(p_ref, xd, info_scale=float(head_dim), amp=True)
    else:
        out_ref = ko.diag_layer(p_ref, xd, amp=True)
    xg = x.to(dev).requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out, _, _ = layer(xg)
    assert out.dtype == torch.bfloat16
    _compare_layer(layer, p_ref, xd, xg, out, out_ref, dy)


def test_layer_training_requires_bf16_autocast():
    dev = gpu_or_skip()
    layer = _layer("iso", dev, 2).train()
    with pytest.raises(TypeError, match="autocast"):
        layer(torch.zeros(1, 8, 128, device=dev))


def _tiny_gpt(mixer_type, dev):
    from lit_gpt.config import Config
    from lit_gpt.model import GPT
    cfg = Config(name="tiny", block_size=256, vocab_size=200, padding_multiple=64, gdn2_per_layer=1,
                 mixer_type=mixer_type, n_layer=2, n_head=2, n_embd=128, rotary_percentage=1.0,
                 parallel_residual=False, bias=False, _norm_class="FusedRMSNorm", norm_eps=1e-5,
                 _mlp_class="LLaMAMLP", intermediate_size=96, mamba_init=True, kdn_info_scale=64.0)
    torch.manual_seed(3)
    model = GPT(cfg)
    model.init_weights()
    return cfg, model.to(dev)


def _gpt_grad_names(mixer_type):
    first = "transformer.h.0.attn." + ("qkv_pack.projection_weight" if mixer_type == "iso_kdn" else "q_proj.weight")
    return ["transformer.wte.weight", "transformer.h.0.norm_1.weight", "transformer.h.0.norm_2.weight", first,
            "transformer.h.1.attn.A_log", "transformer.ln_f.weight", "lm_head.weight"]


def test_gpt_fp32_eval_matches_oracle():
    """Two-layer isotropic GPT in fp32 (eval mode, no autocast) against the fp64 oracle GPT with the
    memory scan's one rounding point: the scan takes bf16 operands, so the normalised q, k and v are
    rounded to bf16 at its boundary (``scan_bf16``).  Logits and gradients at 2e-2.  The rounding's own
    effect |oracle_bf16_scan - oracle_fp64| / max|oracle_fp64| is printed beside each measurement (up to
    ~2e-2 on the second layer's A_log gradient: the bf16 operands, not the kernels, set that error)."""
    dev = gpu_or_skip()
    B, T = 1, 100
    log(f"case GPT iso_kdn 2 layers fp32 eval B={B} T={T}")
    cfg, model = _tiny_gpt("iso_kdn", dev)
    model.eval()
    g = torch.Generator().manual_seed(14)
    idx = torch.randint(0, 200, (B, T), generator=g)
    dl = torch.randn(B, T, cfg.padded_vocab_size, generator=g)
    names = _gpt_grad_names("iso_kdn")
    refs = {}
    for scan_bf16 in (False, True):
        p_ref = {k: v.detach().cpu().double().requires_grad_(True) for k, v in model.state_dict().items()}
        lo = ko.gpt_forward(p_ref, idx, n_layer=2, mixer_type="iso_kdn", info_scale=64.0, scan_bf16=scan_bf16)
        refs[scan_bf16] = [lo.detach()] + list(torch.autograd.grad((lo * dl.double()).sum(),
                                                                   [p_ref[n] for n in names]))
    logits = model(idx.to(dev))
    assert logits.dtype == torch.float32
    params = dict(model.named_parameters())
    grads = torch.autograd.grad(logits, [params[n] for n in names], dl.to(dev))
    torch.cuda.synchronize()
    for n, got, exact, ref in zip(["logits"] + names, [logits] + list(grads), refs[False], refs[True]):
        log(f"  ({n}: bf16 scan operands' effect {rel(ref, exact):.3e})")
        _check(n if n == "logits" else f"d {n}", got, ref, TOL_LAYER)


@pytest.mark.parametrize("mixer_type", ["iso_kdn", "diag_kdn"])
def test_gpt_bf16_autocast_matches_oracle(mixer_type):
    """Two-layer GPT under CUDA bf16 autocast (training mode) against the oracle GPT with autocast's
    rounding points, forward and backward (the oracle rounds a bf16 tensor's cotangent to bf16, as
    autograd does): logits and gradients at 2e-2.  The oracle's own autocast effect
    |oracle_amp - oracle_fp64| / max|oracle_fp64| is printed beside each measurement."""
    dev = gpu_or_skip()
    B, T = 1, 100
    log(f"case GPT {mixer_type} 2 layers autocast B={B} T={T}")
    cfg, model = _tiny_gpt(mixer_type, dev)
    model.train()
    g = torch.Generator().manual_seed(13)
    idx = torch.randint(0, 200, (B, T), generator=g)
    dl = torch.randn(B, T, cfg.padded_vocab_size, generator=g).bfloat16().float()
    kw = {"info_scale": 64.0} if mixer_type == "iso_kdn" else {}
    names = _gpt_grad_names(mixer_type)
    refs = {}
    for amp in (False, True):
        p_ref = {k: v.detach().cpu().double().requires_grad_(True) for k, v in model.state_dict().items()}
        lo = ko.gpt_forward(p_ref, idx, n_layer=2, mixer_type=mixer_type, amp=amp, **kw)
        refs[amp] = [lo.detach()] + list(torch.autograd.grad((lo * dl.double()).sum(), [p_ref[n] for n in names]))
    with torch.autocast("cuda", dtype=torch.bfloat16):
        logits = model(idx.to(dev))
    params = dict(model.named_parameters())
    grads = torch.autograd.grad(logits, [params[n] for n in names], dl.to(dev).to(logits.dtype))
    torch.cuda.synchronize()
    for n, got, exact, amp_ref in zip(["logits"] + names, [logits] + list(grads), refs[False], refs[True]):
        log(f"  ({n}: oracle autocast effect {rel(amp_ref, exact):.3e})")
        _check(n if n == "logits" else f"d {n}", got, amp_ref, TOL_LAYER)
