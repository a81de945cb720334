"""GPU parity of the fused diag front half (``diag_kdn_front``: q/k normalisation -> retention
frontend -> vector gain in one op, reference lit_gpt/diag_kdn.py:315-345) against the three separate
ops it replaces (``_diag_kdn_normalize``, ``_diag_kdn_frontend_precumsum_paired``, ``_diag_kdn_gain``),
which the other GPU tests pin to the CPU oracle.

The normalised q/k come from the same kernel (bit-identical).  The fused kernels recompute alpha,
omega and r on the hardware exp2 / log2 / reciprocal (~1 ulp each, branch-free) where the standalone
kernels use the library exp / log and IEEE division, and sum the log-decay prefix and the parameter
gradients in another order (per 16-token tile instead of per 4-token group); alpha = exp(-e^A
softplus(.)) carries a relative error of about e^A softplus(.) ulp.  Tolerances: 2e-5 (max-relative)
for forward values and fp32 gradients; a bf16 gradient (the raw logits', and the key's for bf16 keys)
may differ by one bf16 rounding step where the fp32 values straddle a rounding boundary, so each of its
elements must agree within 2^-7 relative (one bf16 ulp is 2^-8 to 2^-7 of the value) plus 1e-6 of the
tensor's largest element."""
import pytest
import torch

from gpu_util import gpu_or_skip, log, rel

pytestmark = pytest.mark.gpu

TOL_FWD = 2e-5
TOL_GRAD = 2e-5


def _check_grad(name, got, ref):
    assert torch.isfinite(got).all(), name
    if ref.dtype == torch.bfloat16:
        a, b = got.double(), ref.double()
        scale = float(b.abs().max())
        excess = float(((a - b).abs() - (2.0 ** -7 * b.abs() + 1e-6 * scale)).max())
        log(f"  d{name}: max rel {rel(got, ref):.2e} (per element within one bf16 ulp: {excess <= 0})")
        assert excess <= 0, name
    else:
        r = rel(got, ref)
        log(f"  d{name}: {r:.2e}")
        assert r < TOL_GRAD, name


def _inputs(seed, B, T, H, K, dtype, dev, *, prec=None):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=g)
    k = torch.randn(B, T, H, K, generator=g)
    k[0, 0, 0] = 0.0  # a zero key row: the normalisation's clamped branch
    ret = torch.randn(B, T, H, K, generator=g) * 1.5
    ret[..., :3] = 9.0  # strong decay: alpha below the memory path's 1e-6 floor on some channels
    om = torch.randn(B, T, H, K, generator=g)
    rr = torch.randn(B, T, H, generator=g)
    A_log = torch.log(1 + 3 * torch.rand(H, generator=g))
    dt_bias = 0.3 * torch.randn(H, K, generator=g)
    mu_param = torch.randn(H, generator=g)
    to = lambda x, dt: x.to(device=dev, dtype=dt).contiguous()  # noqa: E731
    d = dict(q=to(q, dtype), k=to(k, dtype), retention_raw=to(ret, torch.bfloat16),
             omega_raw=to(om, torch.bfloat16), r_raw=to(rr, torch.bfloat16), A_log=to(A_log, torch.float32),
             dt_bias=to(dt_bias, torch.float32), initial_precision_param=to(mu_param, torch.float32))
    if prec == "bhk":
        d["initial_precision"] = to(0.2 + torch.rand(B, H, K, generator=g), torch.float32)
    elif prec == "h":
        d["initial_precision"] = to(0.2 + torch.rand(H, generator=g), torch.float32)
    cot = [torch.randn(B, T, H, K, generator=g) for _ in range(4)]
    cots = dict(dq_mem=to(cot[0], torch.bfloat16), dk_mem=to(cot[1], torch.bfloat16), dg=to(cot[2], torch.float32),
                dkappa=to(cot[3] * 0.1, torch.float32), dfp=to(torch.randn(B, H, K, generator=g), torch.float32))
    return d, cots


def _separate(inp, final):
    from lit_gpt.kdn_ops.diag_kdn_chunk import (_diag_kdn_frontend_precumsum_paired, _diag_kdn_gain,
                                                _diag_kdn_normalize)
    q_memory, k_gain, k_memory = _diag_kdn_normalize(inp["q"], inp["k"])
    g_cumsum, alpha, omega, r, mu = _diag_kdn_frontend_precumsum_paired(
        inp["retention_raw"], inp["omega_raw"], inp["r_raw"], inp["A_log"], inp["dt_bias"],
        inp["initial_precision_param"])
    prec = inp.get("initial_precision", mu)
    out = _diag_kdn_gain(k_gain, alpha, omega, r, prec, inp["omega_raw"], inp["r_raw"], output_final_state=final)
    if final:
        return q_memory, k_memory, g_cumsum, out[0], out[1]
    return q_memory, k_memory, g_cumsum, out


def _fused(inp, final):
    from lit_gpt.kdn_ops.diag_kdn_chunk import diag_kdn_front
    return diag_kdn_front(inp["q"], inp["k"], inp["retention_raw"], inp["omega_raw"], inp["r_raw"], inp["A_log"],
                          inp["dt_bias"], inp["initial_precision_param"],
                          initial_precision=inp.get("initial_precision"), output_final_state=final)


def _run(fn, inp, cots, final):
    leaves = {k: v.detach().clone().requires_grad_(True) for k, v in inp.items()}
    outs = fn(leaves, final)
    grads_out = [cots["dq_mem"], cots["dk_mem"], cots["dg"], cots["dkappa"]] + ([cots["dfp"]] if final else [])
    names = list(leaves)
    grads = torch.autograd.grad(outs, [leaves[n] for n in names], grad_outputs=grads_out, allow_unused=True)
    return [o.detach() for o in outs], dict(zip(names, grads))


@pytest.mark.parametrize("K,dtype", [(128, torch.bfloat16), (64, torch.bfloat16), (64, torch.float32)])
@pytest.mark.parametrize("T", [1, 15, 16, 64, 130, 300])
def test_front_matches_separate_ops(T, K, dtype):
    dev = gpu_or_skip()
    B, H = 2, 3
    log(f"case diag front T={T} K={K} {dtype}")
    inp, cots = _inputs(T * 7 + K, B, T, H, K, dtype, dev)
    ref_out, ref_g = _run(_separate, inp, cots, False)
    got_out, got_g = _run(_fused, inp, cots, False)
    for name, a, b in zip(("q_memory", "k_memory", "g_cumsum", "kappa"), got_out, ref_out):
        r = rel(a, b)
        log(f"  {name}: {r:.2e}")
        assert r < TOL_FWD, name
    for name in ref_g:
        if ref_g[name] is None:
            assert got_g[name] is None, name
            continue
        _check_grad(name, got_g[name], ref_g[name])


@pytest.mark.parametrize("prec", ["bhk", "h"])
@pytest.mark.parametrize("T", [77, 2100])
def test_front_state_carry_matches_separate_ops(T, prec):
    """An explicit prior precision ([B,H,K] or [H]) with the final precision and its cotangent;
    T = 2100 has 132 sixteen-token tiles, so both carries take the two-level form."""
    dev = gpu_or_skip()
    B, H, K = 2, 2, 128
    log(f"case diag front state carry T={T} prec={prec}")
    inp, cots = _inputs(T + 11, B, T, H, K, torch.bfloat16, dev, prec=prec)
    ref_out, ref_g = _run(_separate, inp, cots, True)
    got_out, got_g = _run(_fused, inp, cots, True)
    for name, a, b in zip(("q_memory", "k_memory", "g_cumsum", "kappa", "final_precision"), got_out, ref_out):
        r = rel(a, b)
        log(f"  {name}: {r:.2e}")
        assert r < TOL_FWD, name
    for name in ref_g:
        if ref_g[name] is None:
            assert got_g[name] is None, name
            continue
        _check_grad(name, got_g[name], ref_g[name])


def test_front_forward_only_equals_training_forward():
    """Without autograd the op skips the saved tile carries; the outputs are the same bits."""
    dev = gpu_or_skip()
    from lit_gpt.kdn_ops.diag_kdn_chunk import diag_kdn_front
    inp, _ = _inputs(5, 2, 200, 3, 128, torch.bfloat16, dev)
    args = [inp[k] for k in ("q", "k", "retention_raw", "omega_raw", "r_raw", "A_log", "dt_bias",
                             "initial_precision_param")]
    with torch.no_grad():
        a = diag_kdn_front(*args)
    b = diag_kdn_front(*[x.detach().clone().requires_grad_(True) for x in args])
    for x, y in zip(a, b):
        assert torch.equal(x, y.detach())


def test_front_batch_split_launch():
    """B*T*H*K above 2^30 elements: the tile kernels run over batch rows in several launches (32-bit
    offsets per launch).  The last batch rows of the split call equal a call on those rows alone,
    bit for bit; the parameter gradients (sums over all rows) equal the sum of the two calls."""
    dev = gpu_or_skip()
    from lit_gpt.kdn_ops.diag_kdn_chunk import diag_kdn_front
    B, T, H, K = 16, 32768, 18, 128  # 1.21e9 elements: launches of 14 + 2 batch rows
    log(f"case diag front batch split B={B} T={T} H={H} K={K}")
    torch.manual_seed(0)
    bf = dict(device=dev, dtype=torch.bfloat16)
    q, k, ret, om = (torch.randn(B, T, H, K, **bf) for _ in range(4))
    rr = torch.randn(B, T, H, **bf)
    A_log = torch.zeros(H, device=dev)
    dt_bias = torch.zeros(H, K, device=dev)
    mu = torch.zeros(H, device=dev)
    dg = torch.randn(B, T, H, K, device=dev)
    dkap = torch.randn(B, T, H, K, device=dev) * 0.1

    def run(sl):
        leaves = [x[sl].detach().contiguous().requires_grad_(True) for x in (q, k, ret, om, rr)]
        params = [x.clone().requires_grad_(True) for x in (A_log, dt_bias, mu)]
        outs = diag_kdn_front(*leaves, *params)
        kap, g = outs[3].detach(), outs[2].detach()
        grads = torch.autograd.grad([outs[2], outs[3]], leaves[1:] + params, grad_outputs=[dg[sl], dkap[sl]])
        return kap, g, grads

    kap_all, g_all, gr_all = run(slice(0, B))
    tail = slice(14, B)
    kap_t, g_t, gr_t = run(tail)
    kap_h, g_h, gr_h = run(slice(0, 14))
    assert torch.equal(kap_all[tail], kap_t) and torch.equal(g_all[tail], g_t)
    for a, b in zip(gr_all[:4], gr_t[:4]):  # dk, dretention, domega, dr of the tail rows
        assert torch.equal(a[tail], b)
    for name, a, b, c in zip(("dA_log", "ddt_bias", "dmu_param"), gr_all[4:], gr_h[4:], gr_t[4:]):
        r = rel(a, b + c)
        log(f"  {name}: {r:.2e}")
        assert r < 1e-5, name
