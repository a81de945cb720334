"""GPU tests of ``KDNDecoder``: prefill with the chunked scan, then one token per step, eagerly and
as a replayed HIP graph.

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
