"""GPU tests of ``KDNDecoder``: prefill with the chunked scan, then one token per step, eagerly and
as a replayed HIP graph; and of ``kdn_gemv``, the decode step's weight-streaming projection
(against an fp64 product of the same bf16 weight: 1e-5 for fp32 activations, 1e-2 for bf16
outputs, over 1-8 rows, odd N, K from 128 to 6144, with and without bias, strided rows).

Each graph replay is checked against the eager decoder's step on the same token (the same
kernels on the same inputs: 1e-5), with the eager decoder's own work and a device
synchronisation between replays, and both against the logits of the whole sequence run at once
(1e-2 for the fp32 isotropic model; 2e-2 for the bf16 diagonal model, whose frontend takes bf16
only).  The decoder's state after the steps matches a prefill of the whole sequence (the first
layer's precision at 1e-4 in fp32, 1e-2 in bf16; deeper layers' gate inputs carry the upstream
layers' output differences, so their precision is held to the logits' tolerance).  A short
no-grad forward, which packs each block's input projections into one GEMM, matches the separate
GEMMs of the long one (1e-3 fp32: the scan's bf16 operands can round a last-bit GEMM difference
either way; 1e-2 bf16).
"""
import pytest
import torch

from gpu_util import gpu_or_skip, log, rel
from test_gpu_model import _tiny_gpt

pytestmark = pytest.mark.gpu


def _check(name, got, ref, tol):
    r = rel(got, ref)
    log(f"  {name}: rel err {r:.3e} (tol {tol:g})")
    assert r <= tol, f"{name}: {r:.3e} > {tol}"


@pytest.mark.parametrize("mixer_type", ["iso_kdn", "diag_kdn"])
def test_graph_decoder_matches_eager_and_full_sequence(mixer_type):
    dev = gpu_or_skip()
    B, prompt, T = 2, 40, 47
    log(f"case decoder {mixer_type} B={B} prompt={prompt} steps={T - prompt}")
    from lit_gpt.decode import KDNDecoder
    cfg, model = _tiny_gpt(mixer_type, dev)
    model.eval()
    tol_full, tol_prec = 1e-2, 1e-4
    if mixer_type == "diag_kdn":  # bf16 projections round differently at M = B than at M = B T
        model = model.to(torch.bfloat16)
        tol_full, tol_prec = 2e-2, 1e-2
    g = torch.Generator().manual_seed(31)
    idx = torch.randint(0, 200, (B, T), generator=g).to(dev)
    with torch.no_grad():
        full = model(idx)
        _, st_full = model(idx[:, :T - 1], return_state=True)
        short = model(idx[:, :20])  # 40 rows: the packed-projection inference path
    # the scan stores q, k, v in bf16, so a last-bit GEMM difference can flip a rounding: 1e-3 fp32
    _check("packed-projection forward vs the separate GEMMs", short, full[:, :20], 1e-3 if tol_full < 2e-2 else 1e-2)
    eager = KDNDecoder(model, B, use_graph=False)
    graph = KDNDecoder(model, B, use_graph=True)
    le = eager.prefill(idx[:, :prompt])
    lg = graph.prefill(idx[:, :prompt])
    _check("prefill logits, graph decoder vs eager decoder", lg, le, 0.0)
    _check("prefill logits vs full sequence", le, full[:, :prompt], tol_full)
    for t in range(prompt, T - 1):
        a = eager.step(idx[:, t]).clone()
        torch.cuda.synchronize()
        b = graph.step(idx[:, t]).clone()
        torch.cuda.synchronize()
        _check(f"step {t}: graph replay vs eager", b, a, 1e-5)
        _check(f"step {t}: graph replay vs full sequence", b, full[:, t], tol_full)
    assert graph.state[0].seen_tokens == T - 1
    for i, (s, f) in enumerate(zip(graph.state, st_full)):
        _check(f"layer {i} memory state vs prefill of the whole sequence", s.memory, f.memory, tol_full)
        # deeper layers' gate inputs carry the upstream layers' output differences
        _check(f"layer {i} precision state vs prefill of the whole sequence", s.precision, f.precision,
               tol_prec if i == 0 else tol_full)


@pytest.mark.parametrize("M,N,K,dtype,has_bias,strided", [
    (1, 7204, 2304, torch.bfloat16, False, False), (2, 33, 128, torch.float32, True, False),
    (3, 2304, 6144, torch.bfloat16, True, True), (5, 1, 2304, torch.float32, False, True),
    (8, 12288, 2304, torch.bfloat16, False, False), (8, 300, 128, torch.float32, True, False),
    (1, 2304, 128, torch.bfloat16, True, "offset"), (1, 2304, 7208, torch.bfloat16, False, False),
    (4, 2304, 40, torch.bfloat16, True, False), (2, 17, 8, torch.float32, False, True),
    (7, 513, 1160, torch.float32, True, False)])
def test_gemv_matches_fp64(M, N, K, dtype, has_bias, strided):
    dev = gpu_or_skip()
    log(f"case gemv M={M} N={N} K={K} {dtype} bias={has_bias} strided={strided}")
    from lit_gpt.kdn_ops.step import kdn_gemv
    g = torch.Generator().manual_seed(M * 1000 + N)
    W = (torch.randn(N, K, generator=g) / K ** 0.5).bfloat16()
    bias = torch.randn(N, generator=g).bfloat16() if has_bias else None
    x = torch.randn(M, 2 * K if strided else K, generator=g).to(dtype)
    if strided == "offset":
        x = x[:, 4:K + 4]  # one row at an 8-byte offset, as a packed projection's split leaves it
    elif strided:
        x = x[:, :K]  # rows 2K elements apart
    ref = x.double() @ W.double().T + (bias.double() if has_bias else 0.0)
    y = kdn_gemv(x.to(dev), W.to(dev), bias.to(dev) if has_bias else None)
    torch.cuda.synchronize()
    assert y.shape == (M, N) and y.dtype == dtype
    _check("y", y, ref, 1e-5 if dtype == torch.float32 else 1e-2)



@pytest.mark.parametrize("M,N,K,dtype,has_bias", [
    (1, 7208, 2304, torch.bfloat16, False), (3, 100, 200, torch.bfloat16, True), (8, 513, 1160, torch.float32, True),
    (2, 2304, 128, torch.float32, False)])
def test_gated_gemv_is_swiglu_gate(M, N, K, dtype, has_bias):
    # the fused SwiGLU gate over a packed [w1; w2] weight against fp64 silu(x w1^T + b1) * (x w2^T + b2)
    dev = gpu_or_skip()
    log(f"case gated gemv M={M} N={N} K={K} {dtype} bias={has_bias}")
    from lit_gpt.kdn_ops.step import kdn_gemv
    g = torch.Generator().manual_seed(M * 7 + N)
    W = (torch.randn(2 * N, K, generator=g) / K ** 0.5).bfloat16()
    bias = torch.randn(2 * N, generator=g).bfloat16() if has_bias else None
    x = torch.randn(M, K, generator=g).to(dtype)
    h = x.double() @ W.double().T + (bias.double() if has_bias else 0.0)
    ref = torch.nn.functional.silu(h[:, :N]) * h[:, N:]
    y = kdn_gemv(x.to(dev), W.to(dev), bias.to(dev) if has_bias else None, gated=True)
    torch.cuda.synchronize()
    assert y.shape == (M, N) and y.dtype == dtype
    _check("y", y, ref, 1e-5 if dtype == torch.float32 else 1e-2)


@pytest.mark.parametrize("B,D,dtype,wdtype", [(1, 6912, torch.bfloat16, torch.bfloat16), (3, 24, torch.float32, torch.float32),
                                             (2, 136, torch.bfloat16, torch.float32)])
def test_short_conv_step_matches_conv_of_tail_and_token(B, D, dtype, wdtype):
    # the single-token step equals the fixed-length convolution of [tail, x] at its last token
    # (same summation order: bit-identical), and the tail advances to [tail_1, tail_2, x]
    dev = gpu_or_skip()
    log(f"case short_conv_step B={B} D={D} {dtype} w={wdtype}")
    from lit_gpt.kdn_ops.short_conv import _conv_fwd, short_conv_step
    g = torch.Generator().manual_seed(B * 100 + D)
    tail = torch.randn(B, 3, D, generator=g).to(dtype).to(dev)
    xp = torch.randn(B, 1, D + 8, generator=g).to(dtype).to(dev)
    x = xp[..., :D]  # batch stride D + 8, as a packed projection's split leaves it
    w = torch.randn(D, 4, generator=g).to(wdtype).to(dev)
    want = _conv_fwd(torch.cat([tail, x], 1).contiguous(), w)[:, 3:]
    new_tail = torch.cat([tail[:, 1:], x], 1)
    y = short_conv_step(x, tail, w)
    torch.cuda.synchronize()
    assert torch.equal(y, want)
    assert torch.equal(tail, new_tail)


@pytest.mark.parametrize("B", [1, 3])
def test_iso_layer_decode_step_uses_single_token_convolution(B, monkeypatch):
    """At the iso_kdn_1.3B layer width (2304, 18 x 128 heads, bf16, eval, no_grad) a one-token call on
    an in-place state convolves through ``short_conv_step`` (the packed projection's rows are padded to
    a multiple of 8, so its q|k|v slice is aligned for every batch row), and the decoded outputs match
    the whole sequence run at once (2e-2, bf16)."""
    dev = gpu_or_skip()
    log(f"case iso layer decode at width 2304, B={B}: single-token convolution kernel taken")
    from lit_gpt import iso_kdn
    from lit_gpt.kdn_state import KDNLayerState
    torch.manual_seed(7)
    layer = iso_kdn.IsotropicKalmanDeltaNetwork(hidden_size=2304, head_dim=128, num_heads=18)
    layer = layer.to(dev).to(torch.bfloat16).eval()
    calls = []
    real = iso_kdn.short_conv_step

    def counted(*args, **kwargs):
        calls.append(args[0].shape)
        return real(*args, **kwargs)

    monkeypatch.setattr(iso_kdn, "short_conv_step", counted)
    g = torch.Generator().manual_seed(8)
    T, pre = 12, 8
    x = torch.randn(B, T, 2304, generator=g).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        full, _, _ = layer(x, use_cache=True)
        _, _, st = layer(x[:, :pre], use_cache=True)
        st = KDNLayerState(tuple(c.clone() for c in st.conv), st.memory.clone(), st.precision.clone(),
                           st.seen_tokens, inplace=True)
        outs = []
        for t in range(pre, T):
            o, _, st2 = layer(x[:, t:t + 1], past_key_values=st, use_cache=True)
            assert st2 is st
            outs.append(o)
    torch.cuda.synchronize()
    assert len(calls) == T - pre, f"short_conv_step ran {len(calls)} times for {T - pre} decode steps"
    _check("decoded steps vs whole sequence", torch.cat(outs, 1), full[:, pre:], 2e-2)
