"""The allocation-free iso gain forward (``kdn_iso_gain_fwd_noalloc``) against ``kdn_iso_gain_fwd``
through the C ABI: the same kernels on the same inputs, so beta, p_prev and the final precision are
bit-identical.  Two calls in a row on the library's fixed workspace, the second with a smaller input
(and the [B,H] precision mode), then a third identical to the first; a size beyond the fixed workspace
is rejected on the host with KDN_ERR_ARG before any launch.  Under HIP graph capture (after a first
eager call on the device, which looks up the fixed array's address): replays, with eager calls of
other sizes on the same array between them, are bit-identical to ``kdn_iso_gain_fwd``."""
import pytest
import torch
import torch.nn.functional as F

from gpu_util import gpu_or_skip, log

pytestmark = pytest.mark.gpu


def _inputs(B, T, H, seed, dev, prec_mode):
    g = torch.Generator().manual_seed(seed)
    a = torch.sigmoid(2 + 0.5 * torch.randn(B, T, H, generator=g)) ** 2
    omega = F.softplus(torch.randn(B, T, H, generator=g))
    r = 0.01 + F.softplus(torch.randn(B, T, H, generator=g))
    mu = (0.5 + torch.rand(H, generator=g)) if prec_mode == 0 else (0.5 + torch.rand(B, H, generator=g))
    return [x.to(dev).contiguous() for x in (a, omega, r, mu)]


def _run(name, B, T, H, xs, prec_mode, s, dev):
    from lit_gpt.kdn_ops import _lib
    a, omega, r, mu = xs
    beta = torch.full((B, T, H), float("nan"), device=dev)
    p_prev = torch.full((B, T, H), float("nan"), device=dev)
    fprec = torch.full((B, H), float("nan"), device=dev)
    stream = _lib.stream_of(a)
    if name == "kdn_iso_gain_fwd":
        nbytes = _lib.size("kdn_iso_gain_workspace_size", B, T, H)
        ws = torch.empty((nbytes,), device=dev, dtype=torch.uint8)
        _lib.call(name, _lib.ptr(a), _lib.ptr(omega), _lib.ptr(r), _lib.ptr(mu), prec_mode, B, T, H, s,
                  _lib.ptr(beta), _lib.ptr(p_prev), _lib.ptr(fprec), _lib.ptr(ws), nbytes, stream)
    else:
        _lib.call(name, _lib.ptr(a), _lib.ptr(omega), _lib.ptr(r), _lib.ptr(mu), prec_mode, B, T, H, s,
                  _lib.ptr(beta), _lib.ptr(p_prev), _lib.ptr(fprec), stream)
    torch.cuda.synchronize()
    return beta, p_prev, fprec


def test_noalloc_gain_equals_workspace_gain_on_consecutive_calls():
    dev = gpu_or_skip()
    cases = [(4, 4096, 18, 0, 1.0, 1), (2, 300, 5, 1, 0.5, 2), (4, 4096, 18, 0, 1.0, 1)]
    for B, T, H, prec_mode, s, seed in cases:
        log(f"case noalloc iso gain B={B} T={T} H={H} prec_mode={prec_mode} s={s}")
        xs = _inputs(B, T, H, seed, dev, prec_mode)
        want = _run("kdn_iso_gain_fwd", B, T, H, xs, prec_mode, s, dev)
        got = _run("kdn_iso_gain_fwd_noalloc", B, T, H, xs, prec_mode, s, dev)
        for n, x, y in zip(("beta", "p_prev", "final precision"), got, want):
            assert torch.isfinite(y).all(), n
            assert torch.equal(x, y), f"{n}: max diff {float((x - y).abs().max()):.3e}"
        log("  bit-identical")


def test_noalloc_gain_rejects_sizes_beyond_its_workspace():
    dev = gpu_or_skip()
    from lit_gpt.kdn_ops import _lib
    B, T, H = 183, 4096, 18  # B * H * ceil(T / 64) * 20 bytes = 4,216,320 > 4 MiB
    log(f"case noalloc iso gain oversize B={B} T={T} H={H}: host-side rejection")
    assert B * H * (T // 64) * 20 > 4 << 20
    xs = _inputs(B, T, H, 3, dev, 0)
    with pytest.raises(RuntimeError, match="invalid argument"):
        _run("kdn_iso_gain_fwd_noalloc", B, T, H, xs, 0, 1.0, dev)
    # the largest batch that fits (4,193,280 bytes) still runs and matches
    B = 182
    assert B * H * (T // 64) * 20 <= 4 << 20
    xs = _inputs(B, T, H, 4, dev, 0)
    want = _run("kdn_iso_gain_fwd", B, T, H, xs, 0, 1.0, dev)
    got = _run("kdn_iso_gain_fwd_noalloc", B, T, H, xs, 0, 1.0, dev)
    for x, y in zip(got, want):
        assert torch.equal(x, y)


def test_noalloc_gain_under_graph_capture():
    dev = gpu_or_skip()
    from lit_gpt.kdn_ops import _lib
    B, T, H, s = 4, 4096, 18, 1.0
    log(f"case noalloc iso gain captured in a HIP graph B={B} T={T} H={H}, 3 replays")
    xs = _inputs(B, T, H, 7, dev, 0)
    want = _run("kdn_iso_gain_fwd", B, T, H, xs, 0, s, dev)
    _run("kdn_iso_gain_fwd_noalloc", B, T, H, xs, 0, s, dev)  # first call on the device: outside capture
    a, omega, r, mu = xs
    outs = [torch.empty((B, T, H), device=dev), torch.empty((B, T, H), device=dev), torch.empty((B, H), device=dev)]
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            _lib.call("kdn_iso_gain_fwd_noalloc", _lib.ptr(a), _lib.ptr(omega), _lib.ptr(r), _lib.ptr(mu), 0, B, T,
                      H, s, _lib.ptr(outs[0]), _lib.ptr(outs[1]), _lib.ptr(outs[2]), _lib.stream_of(a))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    other = _inputs(2, 300, 5, 8, dev, 1)
    for rep in range(3):
        for x in outs:
            x.fill_(float("nan"))
        # an eager call of another size on the same fixed array between replays
        _run("kdn_iso_gain_fwd_noalloc", 2, 300, 5, other, 1, 0.5, dev)
        graph.replay()
        torch.cuda.synchronize()
        for n, x, y in zip(("beta", "p_prev", "final precision"), outs, want):
            assert torch.equal(x, y), f"replay {rep} {n}: max diff {float((x - y).abs().max()):.3e}"
        log(f"  replay {rep}: bit-identical")
