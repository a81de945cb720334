"""The overlapped schedule of the memory-scan backward (kdn_mem_bwd with stage bits 0 and 1 in one
call): with one chunk group the reverse state pass runs in two segments, and chunk-backward tasks of
the first segment's chunks run on a second stream while the second segment runs, in one launch that
starts after a 3 us bounded wait (so the second segment's workgroups take the CUs the first one
frees); the remaining tasks run at full width after the pass.

The state gradient crosses the segment boundary in fp32 and every kernel computes what it computes
in the serial schedule, so every output must be bit-identical to separate calls (reverse pass, then
chunk backward), which the other memory-scan tests pin to the fp64 oracle.  Shapes have B*H large
enough for one chunk group (checked): on 256 CUs, 33 chunks (7 in the first segment, 448 side tasks)
and the benchmark's 64 chunks (13; 896 side tasks), as the library's plan_bwd_overlap sizes them for
144 state workgroups and 112 idle CUs, with a ragged last chunk,
a chunk taken by the exact path, a final-state cotangent and the initial-state gradient; iso (beta,
bf16 dO) and diag (kappa, fp32 dO).

The forward has the same kind of schedule (kdn_mem_fwd with stage bits 0, 1 and 2 in one call): the
intra-chunk build of the first chunk range, then that range's state pass beside the second range's
build on the second stream, then the second range's pass from the state carried in fp32.  Its output,
final state and every intermediate the backward reads must equal the separate calls' bit for bit, with
and without an initial state, for training and for a no-backward forward, and under graph capture.
"""
import pytest
import torch

from gpu_util import gpu_or_skip, log

pytestmark = pytest.mark.gpu
CHUNK = 64


def _inputs(dev, seed, B, T, H, K, V, diag, extreme):
    g = torch.Generator(device=dev).manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=g, device=dev)  # noqa: E731
    q = torch.nn.functional.normalize(rn(B, T, H, K), dim=-1).bfloat16()
    k = torch.nn.functional.normalize(rn(B, T, H, K), dim=-1).bfloat16()
    v = rn(B, T, H, V).bfloat16()
    ell = (-0.13 + 0.05 * rn(B, T, H, K)).clamp(max=0.0)
    if extreme:  # one chunk of one head beyond the factored range
        ell[0, 64:128, 0] = (-8.0 + 2.0 * rn(64, K)).clamp(max=0.0)
    G = torch.cat([ell[:, c:c + CHUNK].cumsum(1) for c in range(0, T, CHUNK)], 1) / 0.6931471805599453
    if diag:
        kap = 0.5 * torch.rand(B, T, H, K, generator=g, device=dev) * k.float()
        do = rn(B, T, H, V)
    else:
        kap = 0.2 + 0.8 * torch.rand(B, T, H, generator=g, device=dev)
        do = rn(B, T, H, V).bfloat16()
    dht = 0.1 * rn(B, H, K, V)
    return q, k, v, G.contiguous(), kap.contiguous(), do, dht


@pytest.mark.parametrize("B,T,H,variant,extreme", [
    (2, 2048 + 37, 36, "iso", True),   # 33 chunks
    (4, 4096, 18, "iso", False),       # 64 chunks (the benchmark shape)
    (4, 4096, 18, "diag", True),
])
def test_overlapped_backward_is_bit_identical(B, T, H, variant, extreme):
    dev = gpu_or_skip()
    from lit_gpt.kdn_ops import _memscan
    K = V = 128
    diag = variant == "diag"
    assert _memscan.state_groups(B, T, H, K, V) == 1, "shape must run one chunk group"
    log(f"case overlapped-bwd {variant} B={B} T={T} H={H} extreme={extreme}")
    q, k, v, G, kap, do, dht = _inputs(dev, 11 + T + H, B, T, H, K, V, diag, extreme)
    scale = K ** -0.5
    out_dtype = torch.float32 if diag else torch.bfloat16
    _, saved, _ = _memscan.mem_fwd(q, k, kap, not diag, v, G, scale, out_dtype=out_dtype)
    runs = []
    for overlap in (False, True, True):  # twice overlapped: the side stream's events are reused
        runs.append(_memscan.mem_bwd(q, k, kap, not diag, v, G, saved, scale, do, d_final_state=dht,
                                     need_initial_state_grad=True, overlap=overlap))
    torch.cuda.synchronize()
    names = ("dq", "dk", "dv", "dkappa" if diag else "dbeta", "dg", "d initial state")
    for run in runs[1:]:
        for name, a, b in zip(names, runs[0], run):
            assert torch.isfinite(a).all(), name
            assert torch.equal(a, b), f"{name}: overlapped schedule differs from the serial one"
    log("  bit-identical")


def test_overlapped_backward_under_graph_capture():
    """The overlapped backward captured into a HIP graph (the second stream forks from and joins the
    capturing stream): every replay, with eager work and synchronisations between them, equals the
    eager call bit for bit.  The side queue is made by the eager calls first; a first call inside
    a capture takes the serial schedule instead (stream and event creation are not capturable)."""
    dev = gpu_or_skip()
    from lit_gpt.kdn_ops import _memscan
    B, T, H, K = 4, 4096, 18, 128
    assert _memscan.state_groups(B, T, H, K, K) == 1
    log(f"case overlapped-bwd graph capture iso B={B} T={T} H={H}")
    q, k, v, G, kap, do, dht = _inputs(dev, 3, B, T, H, K, K, False, False)
    scale = K ** -0.5
    _, saved, _ = _memscan.mem_fwd(q, k, kap, True, v, G, scale, out_dtype=torch.bfloat16)
    call = lambda: _memscan.mem_bwd(q, k, kap, True, v, G, saved, scale, do, d_final_state=dht,  # noqa: E731
                                    need_initial_state_grad=True, overlap=True)
    eager = call()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call()
    names = ("dq", "dk", "dv", "dbeta", "dg", "d initial state")
    for rep in range(3):
        noise = torch.randn(1 << 20, device=dev).sum()  # eager work between replays
        again = call()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        for name, a, b, c in zip(names, eager, out, again):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager call"
            assert torch.equal(a, c), f"{name}: eager call {rep} differs"
    log("  replays bit-identical")


@pytest.mark.parametrize("B,T,H,variant,extreme", [
    (2, 2048 + 37, 36, "iso", True),   # 33 chunks, a ragged last chunk, a chunk for the exact path
    (4, 4096, 18, "iso", False),       # the benchmark shape
    (4, 4096, 18, "diag", True),
])
def test_overlapped_forward_is_bit_identical(B, T, H, variant, extreme):
    dev = gpu_or_skip()
    from lit_gpt.kdn_ops import _memscan
    K = V = 128
    diag = variant == "diag"
    assert _memscan.state_groups(B, T, H, K, V) == 1, "shape must run one chunk group"
    log(f"case overlapped-fwd {variant} B={B} T={T} H={H} extreme={extreme}")
    q, k, v, G, kap, do, dht = _inputs(dev, 5 + T + H, B, T, H, K, V, diag, extreme)
    h0 = 0.5 * dht
    scale = K ** -0.5
    out_dtype = torch.float32 if diag else torch.bfloat16
    names = ("dq", "dk", "dv", "dkappa" if diag else "dbeta", "dg", "d initial state")
    for init in (None, h0):
        for need_backward in (True, False):
            runs = [_memscan.mem_fwd(q, k, kap, not diag, v, G, scale, initial_state=init, output_final_state=True,
                                     out_dtype=out_dtype, need_backward=need_backward, overlap=ov)
                    for ov in (False, True, True)]  # twice overlapped: the side stream's events are reused
            # what the backward reads of each forward's saved intermediates: its gradients (serial schedule)
            grads = [_memscan.mem_bwd(q, k, kap, not diag, v, G, s, scale, do, d_final_state=dht,
                                      need_initial_state_grad=True, overlap=False) for _, s, _ in runs] \
                if need_backward else None
            torch.cuda.synchronize()
            o0, _, f0 = runs[0]
            assert torch.isfinite(o0.float()).all() and torch.isfinite(f0).all()
            for i, (o, _, f) in enumerate(runs[1:], 1):
                assert torch.equal(o, o0), "output differs from the serial schedule"
                assert torch.equal(f, f0), "final state differs from the serial schedule"
                if grads is not None:
                    for name, a, b in zip(names, grads[0], grads[i]):
                        assert torch.equal(a, b), f"{name} from the overlapped forward's saved state differs"
    log("  bit-identical")


def test_overlapped_forward_under_graph_capture():
    """The overlapped forward captured into a HIP graph: every replay, with eager work and
    synchronisations between them, equals the eager call bit for bit."""
    dev = gpu_or_skip()
    from lit_gpt.kdn_ops import _memscan
    B, T, H, K = 4, 4096, 18, 128
    assert _memscan.state_groups(B, T, H, K, K) == 1
    log(f"case overlapped-fwd graph capture iso B={B} T={T} H={H}")
    q, k, v, G, kap, _do, dht = _inputs(dev, 9, B, T, H, K, K, False, False)
    scale = K ** -0.5
    call = lambda: _memscan.mem_fwd(q, k, kap, True, v, G, scale, initial_state=dht,  # noqa: E731
                                    output_final_state=True, out_dtype=torch.bfloat16, overlap=True)
    eager = call()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call()
    for rep in range(3):
        noise = torch.randn(1 << 20, device=dev).sum()  # eager work between replays
        again = call()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        for name, a, b, c in zip(("o", "final state"), eager[::2], out[::2], again[::2]):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager call"
            assert torch.equal(a, c), f"{name}: eager call {rep} differs"
    log("  replays bit-identical")


@pytest.mark.parametrize("variant,norm", [("iso", True), ("iso", False), ("diag", False)])
def test_exact_stages_in_one_launch_equal_separate_calls(variant, norm, monkeypatch):
    """kdn_mem_bwd with stage bits 2 and 3 in one call runs each flagged chunk's exact solves, its exact
    gradients and (with the in-op L2 norm) the norm's backward of its q, k rows in one launch; separate
    calls (bit 2, then bit 3) run them as separate kernels.  On inputs with a chunk taken by the exact
    path (a ragged last chunk too) every gradient must be bit-identical."""
    dev = gpu_or_skip()
    from lit_gpt.kdn_ops import _memscan
    B, T, H, K = 2, 2048 + 37, 3, 128
    diag = variant == "diag"
    log(f"case exact stages one launch vs separate {variant} norm={norm} B={B} T={T} H={H}")
    q, k, v, G, kap, do, dht = _inputs(dev, 77, B, T, H, K, K, diag, True)
    rs = {}
    if norm:  # raw rows the op normalises itself
        q, k = (2.5 * q.float()).bfloat16(), (0.75 * k.float()).bfloat16()
        rs = {"q_rstd": torch.empty(B, T, H, device=dev), "k_rstd": torch.empty(B, T, H, device=dev)}
    scale = K ** -0.5
    _, saved, _ = _memscan.mem_fwd(q, k, kap, not diag, v, G, scale, output_final_state=True,
                                   out_dtype=torch.float32 if diag else torch.bfloat16, **rs)

    def run():
        return _memscan.mem_bwd(q, k, kap, not diag, v, G, saved, scale, do, d_final_state=dht,
                                need_initial_state_grad=True, overlap=False, **rs)

    one = run()
    monkeypatch.setattr(_memscan, "BWD_STAGES", ((1, "mem_state_bwd"), (2, "mem_bwd_chunk"),
                                                 (4, "mem_bwd_solve_exact"), (8, "mem_bwd_contrib_exact")))
    separate = run()
    torch.cuda.synchronize()
    names = ("dq", "dk", "dv", "dkappa" if diag else "dbeta", "dg", "d initial state")
    for name, a, b in zip(names, one, separate):
        assert torch.isfinite(a.float()).all(), name
        assert torch.equal(a, b), f"{name}: one launch differs from the separate exact stages"
    log("  bit-identical")
