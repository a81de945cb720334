"""GPU parity of the state-carry path (segmented prefill and token-by-token decode).

* Isotropic gain continuation: a sequence split in two, the second part starting from the first
  part's final precision ([B,H] initial precision), against the fp64 tokenwise gain of the whole
  sequence: beta and final precision at 1e-5, gradients (through the carried precision and the
  final precision's cotangent) at 1e-4.
* ``kdn_mem_step``: several single-token steps from a random fp32 state against the oracle's
  tokenwise recurrence (``memory_tokenwise``, fed the same rounded inputs, with the FLA l2norm of
  q, k for the isotropic form): outputs and state at 1e-4 (fp32 outputs) / 1e-2 (bf16 outputs).
  ``kdn_kalman_step`` (gain and memory in one launch) likewise, from a random precision too,
  against the tokenwise gains feeding the same recurrence: outputs, state, precision at 1e-4.
* Layers in eval mode (isotropic fp32; diagonal under bf16 autocast, its frontend taking bf16
  only): full sequence vs a chunked prefill, a second chunked segment and single-token steps,
  each against the oracle layer of the whole sequence (2e-2, or the autocast noise floor) and
  against the GPU full-sequence run (1e-2; the paths round q, k, v at different points); states.
* Layers in training mode under bf16 autocast: two differentiable segments with the state carried
  between them, output and every gradient (crossing the carried memory, precision and convolution
  inputs) against the GPU run of the whole sequence at 1e-2 and against the autocast oracle at
  2e-2 (the oracle rounds bf16 cotangents as autograd does).
* GPT: prefill then decode under no_grad against the oracle GPT of the whole sequence.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from gpu_util import gpu_or_skip, log, rel
from oracle import kdn_oracle as ko
from test_gpu_model import _layer, _oracle_params, _tiny_gpt

pytestmark = pytest.mark.gpu
LN2 = math.log(2.0)


def _check(name, got, ref, tol):
    r = rel(got, ref)
    log(f"  {name}: rel err {r:.3e} (tol {tol:g})")
    assert r <= tol, f"{name}: {r:.3e} > {tol}"


def _iso_gain_ref(a, omega, r, mu, s):
    """Production iso gain on unit keys from p_0 = 1/mu (mu [H] or [B,H]); returns (beta, 1/p_T).
    The oracle's golden-pinned tokenwise gain."""
    return ko.iso_gain_unit_key(a, omega, r, mu, posterior_scale=s, output_final_state=True)


@pytest.mark.parametrize("T1,T2,info_scale", [(70, 80, None), (64, 1, 64.0), (1, 130, None)])
def test_iso_gain_continuation(T1, T2, info_scale):
    dev = gpu_or_skip()
    log(f"case iso gain continuation T1={T1} T2={T2} info_scale={info_scale}")
    from lit_gpt.kdn_ops.iso_kdn_chunk import iso_kdn_gain
    B, H, K = 3, 4, 128
    T = T1 + T2
    g = torch.Generator().manual_seed(T1 * 1000 + T2)
    a = torch.sigmoid(2 + 0.5 * torch.randn(B, T, H, generator=g)) ** 2
    omega = F.softplus(torch.randn(B, T, H, generator=g))
    r = 0.01 + F.softplus(torch.randn(B, T, H, generator=g))
    mu = 0.5 + torch.rand(H, generator=g)
    db = torch.randn(B, T, H, generator=g)
    dfp = torch.randn(B, H, generator=g)
    s = (K if info_scale is None else info_scale) / K
    leaves = [x.double().requires_grad_(True) for x in (a, omega, r, mu)]
    beta_ref, fp_ref = _iso_gain_ref(*leaves, s)
    gref = torch.autograd.grad((beta_ref * db.double()).sum() + (fp_ref * dfp.double()).sum(), leaves)
    gl = [x.to(dev).requires_grad_(True) for x in (a, omega, r, mu)]
    beta1, fp1 = iso_kdn_gain(gl[0][:, :T1], gl[1][:, :T1], gl[2][:, :T1], gl[3], head_dim=K,
                              info_scale=info_scale, output_final_state=True)
    assert fp1.shape == (B, H)
    beta2, fp2 = iso_kdn_gain(gl[0][:, T1:], gl[1][:, T1:], gl[2][:, T1:], fp1, head_dim=K,
                              info_scale=info_scale, output_final_state=True)
    beta = torch.cat([beta1, beta2], 1)
    gg = torch.autograd.grad((beta * db.to(dev)).sum() + (fp2 * dfp.to(dev)).sum(), gl)
    _check("beta", beta, beta_ref, 1e-5)
    _check("final precision", fp2, fp_ref, 1e-5)
    for name, x, y in zip(("da", "domega", "dr", "dmu"), gg, gref):
        _check(name, x, y, 1e-4)


@pytest.mark.parametrize("variant,K,V,dtype,out_dtype", [
    ("iso", 128, 128, torch.bfloat16, torch.float32), ("iso", 64, 128, torch.float32, torch.float32),
    ("iso", 128, 64, torch.bfloat16, torch.bfloat16), ("diag", 128, 128, torch.bfloat16, torch.float32),
    ("diag", 64, 64, torch.float32, torch.float32), ("diag", 128, 64, torch.bfloat16, torch.bfloat16)])
def test_memory_step_matches_tokenwise(variant, K, V, dtype, out_dtype):
    dev = gpu_or_skip()
    log(f"case mem step {variant} K={K} V={V} in={dtype} out={out_dtype}")
    from lit_gpt.kdn_ops.step import kdn_memory_step
    B, H, steps = 3, 5, 6
    g = torch.Generator().manual_seed(K + V + (0 if variant == "iso" else 1))
    q = 2.0 * torch.randn(B, steps, H, K, generator=g)
    k = 2.0 * torch.randn(B, steps, H, K, generator=g)
    if variant == "diag":  # the diagonal form takes normalised q, k
        q, k = ko.diag_normalize(q), ko.diag_normalize(k)
    q, k = q.to(dtype), k.to(dtype)
    v = torch.randn(B, steps, H, V, generator=g).to(dtype)
    g2 = ((-0.13 + 0.05 * torch.randn(B, steps, H, K, generator=g)).clamp(max=0.0) / LN2).float()
    S0 = torch.randn(B, H, K, V, generator=g)
    qd, kd, vd = q.double(), k.double(), v.double()
    if variant == "iso":
        beta = 0.2 + 0.8 * torch.rand(B, steps, H, generator=g)
        qd, kd = ko.l2norm_fla(qd), ko.l2norm_fla(kd)
        kap_ref = beta.double()[..., None] * kd
    else:
        kappa = 0.5 * torch.rand(B, steps, H, K, generator=g) * k.float()
        kap_ref = kappa.double()
    o_ref, S_ref = ko.memory_tokenwise(qd, kd, vd, (g2.double() * LN2).exp(), kap_ref, scale=K ** -0.5,
                                       initial_state=S0.double())
    state = S0.to(dev).contiguous()
    outs = []
    for t in range(steps):
        sl = slice(t, t + 1)
        kw = {"beta": beta[:, sl].to(dev)} if variant == "iso" else {"kappa": kappa[:, sl].to(dev)}
        outs.append(kdn_memory_step(q[:, sl].to(dev), k[:, sl].to(dev), v[:, sl].to(dev), g2[:, sl].to(dev),
                                    state=state, out_dtype=out_dtype, **kw))
    o = torch.cat(outs, 1)
    torch.cuda.synchronize()
    assert o.dtype == out_dtype
    _check("o", o, o_ref, 1e-4 if out_dtype == torch.float32 else 1e-2)
    _check("state", state, S_ref, 1e-4)


@pytest.mark.parametrize("variant,K,V,dtype", [("iso", 128, 128, torch.bfloat16), ("iso", 64, 128, torch.float32),
                                               ("diag", 128, 128, torch.bfloat16), ("diag", 64, 64, torch.float32)])
def test_kalman_step_matches_tokenwise(variant, K, V, dtype):
    """``kdn_kalman_step`` (the single-token gain from the carried precision, then the memory
    update, in one launch), six steps from a random state and precision, against the tokenwise
    gain (iso: the production unit-key form; diag: ``diag_gain_tokenwise``) feeding
    ``memory_tokenwise``: outputs, state and final precision at 1e-4."""
    dev = gpu_or_skip()
    log(f"case kalman step {variant} K={K} V={V} in={dtype}")
    from lit_gpt.kdn_ops.step import kdn_kalman_step
    B, H, steps = 2, 3, 6
    g = torch.Generator().manual_seed(7 * K + V + (0 if variant == "iso" else 1))
    q = 2.0 * torch.randn(B, steps, H, K, generator=g)
    k = 2.0 * torch.randn(B, steps, H, K, generator=g)
    if variant == "diag":
        q, k = ko.diag_normalize(q), ko.diag_normalize(k)
    k_gain = k.clone()  # the diagonal gain's fp32 key
    q, k = q.to(dtype), k.to(dtype)
    v = torch.randn(B, steps, H, V, generator=g).to(dtype)
    g2 = ((-0.13 + 0.05 * torch.randn(B, steps, H, K, generator=g)).clamp(max=0.0) / LN2).float()
    S0 = torch.randn(B, H, K, V, generator=g)
    r = 0.01 + F.softplus(torch.randn(B, steps, H, generator=g))
    qd, kd, vd = q.double(), k.double(), v.double()
    if variant == "iso":
        a = torch.sigmoid(2 + 0.5 * torch.randn(B, steps, H, generator=g)) ** 2
        omega = F.softplus(torch.randn(B, steps, H, generator=g))
        c0 = 0.5 + torch.rand(B, H, generator=g)
        qd, kd = ko.l2norm_fla(qd), ko.l2norm_fla(kd)
        beta_ref, c_ref = _iso_gain_ref(a.double(), omega.double(), r.double(), c0.double(), 1.0)
        kap_ref = beta_ref[..., None] * kd
        gain_kw = {"a": a}
    else:
        alpha = torch.sigmoid(2 + 0.5 * torch.randn(B, steps, H, K, generator=g))
        omega = F.softplus(torch.randn(B, steps, H, K, generator=g))
        c0 = 0.3 + torch.rand(B, H, K, generator=g)
        kap_ref, c_ref = ko.diag_gain_tokenwise(k_gain.double(), alpha.double(), omega.double(), r.double(),
                                                info_scale=float(K), initial_precision=c0.double(),
                                                output_final_state=True)
        gain_kw = {"alpha": alpha}
    o_ref, S_ref = ko.memory_tokenwise(qd, kd, vd, (g2.double() * LN2).exp(), kap_ref, scale=K ** -0.5,
                                       initial_state=S0.double())
    state, prec = S0.to(dev).contiguous(), c0.to(dev)
    outs = []
    for t in range(steps):
        sl = slice(t, t + 1)
        kw = {n: x[:, sl].to(dev) for n, x in gain_kw.items()}
        if variant == "diag":
            kw["k_gain"] = k_gain[:, sl].to(dev)
        o, prec = kdn_kalman_step(q[:, sl].to(dev), k[:, sl].to(dev), v[:, sl].to(dev), g2[:, sl].to(dev),
                                  state=state, precision=prec, omega=omega[:, sl].to(dev), r=r[:, sl].to(dev),
                                  info_scale=float(K), out_dtype=torch.float32, **kw)
        outs.append(o)
    torch.cuda.synchronize()
    _check("o", torch.cat(outs, 1), o_ref, 1e-4)
    _check("state", state, S_ref, 1e-4)
    _check("final precision", prec, c_ref, 1e-4)


def _oracle_layer(variant, p, x, head_dim, amp=False):
    if variant == "iso":
        return ko.iso_layer(p, x, info_scale=float(head_dim), amp=amp)
    return ko.diag_layer(p, x, amp=amp)


def _amp_tol(amp_ref, exact):
    """Oracle-side bar under autocast: 2e-2, as without it.  The oracle rounds to bf16 at autocast's
    rounding points; its own autocast effect (amp vs exact) is printed beside the measurement."""
    log(f"  (oracle autocast effect {rel(amp_ref, exact):.3e})")
    return 2e-2


@pytest.mark.parametrize("variant,head_dim", [("iso", 64), ("diag", 64), ("iso", 128), ("diag", 128)])
def test_layer_segments_and_decode_match_full_sequence(variant, head_dim):
    """Isotropic layers run in fp32 eval mode; the diagonal layer's frontend takes bf16 inputs only
    (as the reference's does), so it runs in eval mode under bf16 autocast."""
    dev = gpu_or_skip()
    B, T, cut1, cut2 = 2, 150, 70, 134
    log(f"case {variant} layer state carry eval B={B} T={T} K={head_dim} segments 0:{cut1}:{cut2}:+1")
    layer = _layer(variant, dev, 4, head_dim).eval()
    g = torch.Generator().manual_seed(21)
    x = torch.randn(B, T, 2 * head_dim, generator=g)
    p_ref = _oracle_params(layer)
    amp = variant == "diag"
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=amp):
        out_ref = _oracle_layer(variant, p_ref, x.double(), head_dim, amp=amp)
        tol = _amp_tol(out_ref, _oracle_layer(variant, p_ref, x.double(), head_dim)) if amp else 2e-2
        xg = x.to(dev)
        full, _, st_full = layer(xg, use_cache=True)
        o1, _, st = layer(xg[:, :cut1], use_cache=True)
        o2, _, st = layer(xg[:, cut1:cut2], past_key_values=st, use_cache=True)
        outs = [o1, o2]
        for t in range(cut2, T):
            o, _, st = layer(xg[:, t:t + 1], past_key_values=st, use_cache=True)
            outs.append(o)
        seg = torch.cat(outs, 1)
        plain, _, none = layer(xg)
    torch.cuda.synchronize()
    assert none is None and st.seen_tokens == T and st_full.seen_tokens == T
    _check("full (stateful call)", full, out_ref, tol)
    _check("segmented + decoded", seg, out_ref, tol)
    _check("segmented vs GPU full", seg, full, 1e-2)
    _check("stateful vs plain full call", full, plain, 1e-6)
    _check("memory state", st.memory, st_full.memory, 1e-2)
    # bf16 projections of one token and of a whole segment come from different GEMM kernels and may
    # differ in the last bit under autocast; the fp32 isotropic layer holds the precision to 1e-4
    _check("precision state", st.precision, st_full.precision, 1e-3 if amp else 1e-4)
    for i, (a, b) in enumerate(zip(st.conv, st_full.conv)):
        _check(f"conv state {i}", a, b, 1e-5)


@pytest.mark.parametrize("variant", ["iso", "diag"])
def test_layer_state_carry_gradients_under_autocast(variant):
    """Two differentiable segments with the state carried between them: output and every gradient
    against the same layer run on the whole sequence at once (1e-2: the runs differ only in chunk
    boundaries; this is the carry's contract), and against the autocast oracle of the whole
    sequence at 2e-2.  The oracle rounds to bf16 where autocast stores bf16 tensors, in the forward
    and in the backward (a bf16 tensor's cotangent is bf16)."""
    dev = gpu_or_skip()
    B, T, cut, head_dim = 2, 130, 70, 64
    log(f"case {variant} layer autocast training, two segments carried 0:{cut}:{T}")
    layer = _layer(variant, dev, 5, head_dim).train()
    g = torch.Generator().manual_seed(22)
    x = torch.randn(B, T, 2 * head_dim, generator=g)
    dy = torch.randn(B, T, 2 * head_dim, generator=g).bfloat16().float()
    names = [n for n, _ in layer.named_parameters()]
    refs = {}
    for amp in (False, True):
        p_ref = _oracle_params(layer)
        xd = x.double().requires_grad_(True)
        o = _oracle_layer(variant, p_ref, xd, head_dim, amp=amp)
        refs[amp] = [o.detach()] + list(torch.autograd.grad((o * dy.double()).sum(), [xd] + [p_ref[n] for n in names]))
    params = dict(layer.named_parameters())
    runs = {}
    for mode in ("full", "segments"):
        xg = x.to(dev).requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            if mode == "full":
                out, _, _ = layer(xg)
            else:
                o1, _, st = layer(xg[:, :cut], use_cache=True)
                o2, _, _ = layer(xg[:, cut:], past_key_values=st)
                out = torch.cat([o1, o2], 1)
        grads = torch.autograd.grad(out, [xg] + [params[n] for n in names], dy.to(dev).to(out.dtype))
        runs[mode] = [out.detach()] + list(grads)
    torch.cuda.synchronize()
    for i, n in enumerate(["output", "d hidden"] + [f"d {n}" for n in names]):
        _check(f"{n} segments vs full", runs["segments"][i], runs["full"][i], 1e-2)
        _check(f"{n} segments vs oracle", runs["segments"][i], refs[True][i], 2e-2)


@pytest.mark.parametrize("mixer_type", ["iso_kdn", "diag_kdn"])
def test_gpt_prefill_then_decode_matches_full_sequence(mixer_type):
    dev = gpu_or_skip()
    B, T, prefill = 1, 72, 64
    log(f"case GPT {mixer_type} prefill {prefill} then decode to {T}")
    cfg, model = _tiny_gpt(mixer_type, dev)
    model.eval()
    g = torch.Generator().manual_seed(23)
    idx = torch.randint(0, 200, (B, T), generator=g)
    kw = {"info_scale": 64.0} if mixer_type == "iso_kdn" else {}
    p_ref = {k: v.detach().cpu().double() for k, v in model.state_dict().items()}
    amp = mixer_type == "diag_kdn"  # the diagonal frontend takes bf16 inputs only
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=amp):
        logits_ref = ko.gpt_forward(p_ref, idx, n_layer=2, mixer_type=mixer_type, amp=amp, **kw)
        tol = _amp_tol(logits_ref, ko.gpt_forward(p_ref, idx, n_layer=2, mixer_type=mixer_type, **kw)) if amp else 2e-2
        ig = idx.to(dev)
        full = model(ig)
        lp, st = model(ig[:, :prefill], return_state=True)
        outs = [lp]
        for t in range(prefill, T):
            lt, st = model(ig[:, t:t + 1], state=st, return_state=True)
            outs.append(lt)
        seg = torch.cat(outs, 1)
    torch.cuda.synchronize()
    assert len(st) == 2 and all(s.seen_tokens == T for s in st)
    _check("full", full, logits_ref, tol)
    _check("prefill + decode", seg, logits_ref, tol)
    _check("prefill + decode vs GPU full", seg, full, 1e-2)
