"""The "recompute" backward mode of the memory scan (_memscan.set_backward_mode): the forward keeps
only the op's inputs, as the reference's autograd functions do (iso_kdn_chunk.py:2206,
diag_kdn_chunk.py:3253), and the backward rebuilds the intra-chunk WY factors, A^T and the per-chunk
states from them before its own passes, as the reference re-runs recompute_w_u_fwd and the state
forward (iso_kdn_chunk.py:2101-2140, diag_kdn_chunk.py:3271-3277).

The rebuild runs the forward's kernels on the same inputs, so every gradient must be bit-identical to
the "save" mode's, which the other memory-scan tests pin to the fp64 oracle.  Cases: the isotropic op
with the in-op norm (bf16 q, k) and with fp32 q, k (the separate norm kernels), the diagonal scan
(chunk_kalman); an initial state and a final-state cotangent; a ragged last chunk and a chunk on the
exact per-block path; one chunk group (B*H = 72, the benchmark's width) and the two-level state scan
(B*H = 2, 16 chunk groups), whose rebuilt states come from the combine of the group maps.
"""
import pytest
import torch

from gpu_util import chunk_prefix_base2, gpu_or_skip, log

pytestmark = pytest.mark.gpu
CHUNK = 64


def _inputs(seed, B, T, H, K, V, diag, qk_dtype, extreme):
    g = torch.Generator().manual_seed(seed)
    q = (1.7 * torch.randn(B, T, H, K, generator=g)).to(qk_dtype)
    k = (0.6 * torch.randn(B, T, H, K, generator=g)).to(qk_dtype)
    if diag:
        q = torch.nn.functional.normalize(q.float(), dim=-1).bfloat16()
        k = torch.nn.functional.normalize(k.float(), dim=-1).bfloat16()
    v = torch.randn(B, T, H, V, generator=g).to(torch.bfloat16 if diag else qk_dtype)
    ell = (-0.13 + 0.05 * torch.randn(B, T, H, K, generator=g)).clamp(max=0.0)
    if extreme:  # one chunk beyond the factored range
        ell[:, 64:128] = (-8.0 + 2.0 * torch.randn(B, 64, H, K, generator=g)).clamp(max=0.0)
    G2 = chunk_prefix_base2(ell, CHUNK).float()
    if diag:
        kap = 0.5 * torch.rand(B, T, H, K, generator=g) * k.float()
        do = torch.randn(B, T, H, V, generator=g)
    else:
        kap = 0.2 + 0.8 * torch.rand(B, T, H, generator=g)
        do = torch.randn(B, T, H, V, generator=g).to(qk_dtype)
    h0 = 0.3 * torch.randn(B, H, K, V, generator=g)
    dht = 0.1 * torch.randn(B, H, K, V, generator=g)
    return q, k, v, G2, kap.float(), do, h0, dht


def _grads(variant, dev, tensors, scale):
    from lit_gpt.kdn_ops import diag_kdn_chunk as dk
    from lit_gpt.kdn_ops import iso_kdn_chunk as ik
    q, k, v, G, kap, do, h0, dht = (x.to(dev).contiguous() for x in tensors)
    leaves = [x.clone().requires_grad_(True) for x in (q, k, v, G, kap, h0)]
    if variant == "iso":
        o, ht = ik._chunk_kda_precumsum_paired(leaves[0], leaves[1], leaves[2], leaves[3], leaves[4], scale,
                                               initial_state=leaves[5], output_final_state=True)
    else:
        o, ht = dk.chunk_kalman(leaves[0], leaves[1], leaves[4], leaves[2], leaves[3], scale,
                                initial_state=leaves[5], output_final_state=True)
    grads = torch.autograd.grad([o, ht], leaves, grad_outputs=[do, dht])
    torch.cuda.synchronize()
    return o.detach(), ht.detach(), grads


@pytest.mark.parametrize("B,T,H,variant,qk_dtype,extreme", [
    (2, 2048 + 37, 36, "iso", torch.bfloat16, True),    # one chunk group, in-op norm in the scan
    (1, 300, 2, "iso", torch.float32, True),            # fp32 q, k: the separate norm kernels
    (1, 8192 + 21, 2, "iso", torch.bfloat16, False),    # two-level state scan
    (2, 2048 + 37, 36, "diag", torch.bfloat16, True),
    (1, 8192 + 21, 2, "diag", torch.bfloat16, True),
])
def test_recompute_backward_is_bit_identical(B, T, H, variant, qk_dtype, extreme):
    dev = gpu_or_skip()
    from lit_gpt.kdn_ops import _memscan
    K = V = 128
    log(f"case recompute-bwd {variant} B={B} T={T} H={H} qk={qk_dtype} extreme={extreme} "
        f"groups={_memscan.state_groups(B, T, H, K, V)}")
    tensors = _inputs(5 + T + H, B, T, H, K, V, variant == "diag", qk_dtype, extreme)
    scale = K ** -0.5
    assert _memscan.backward_mode() == "save"
    ref = _grads(variant, dev, tensors, scale)
    prev = _memscan.set_backward_mode("recompute")
    try:
        got = _grads(variant, dev, tensors, scale)
    finally:
        _memscan.set_backward_mode(prev)
    assert torch.equal(ref[0], got[0]) and torch.equal(ref[1], got[1]), "forward outputs differ"
    names = ("dq", "dk", "dv", "dg", "dkappa" if variant == "diag" else "dbeta", "d initial state")
    for name, a, b in zip(names, ref[2], got[2]):
        assert torch.isfinite(a).all(), name
        assert torch.equal(a, b), f"{name}: the recompute mode differs from the save mode"
    log("  bit-identical")


def test_recompute_mode_keeps_no_intermediates():
    """In the recompute mode the autograd graph holds no saved buffer of the scan's intermediates."""
    dev = gpu_or_skip()
    from lit_gpt.kdn_ops import _memscan
    from lit_gpt.kdn_ops import iso_kdn_chunk as ik
    B, T, H, K = 2, 1024, 4, 128
    tensors = _inputs(3, B, T, H, K, K, False, torch.bfloat16, False)
    q, k, v, G, kap = (x.to(dev).contiguous().requires_grad_(True) for x in tensors[:5])
    saved_bytes = _memscan._lib.size("kdn_mem_saved_size", B, T, H, K, K)
    held = {}
    for mode in ("save", "recompute"):
        prev = _memscan.set_backward_mode(mode)
        try:
            torch.cuda.synchronize()
            before = torch.cuda.memory_allocated(dev)
            o = ik._chunk_kda_precumsum_paired(q, k, v, G, kap, K ** -0.5)
            torch.cuda.synchronize()
            held[mode] = torch.cuda.memory_allocated(dev) - before - o.numel() * o.element_size()
            del o
        finally:
            _memscan.set_backward_mode(prev)
    log(f"held by the graph: save {held['save']} B, recompute {held['recompute']} B (saved buffer {saved_bytes} B)")
    assert held["save"] >= saved_bytes
    assert held["recompute"] < saved_bytes // 8
