"""Pin the CPU oracle (oracle/kdn_oracle.py) against the reference's own outputs.

The fixtures in tests/golden/ were written by tests/golden/make_golden.py from the
reference's tokenwise oracles (iso_kdn_naive.py:200-251,376-440 and
diag_kdn_naive.py:217-276,503-567).  A transcription mistake in the restatement
(a dropped 1/K, a swapped alpha/alpha^2, readout before the write) fails here.
"""
import pathlib

import numpy as np
import pytest
import torch

from oracle import kdn_oracle as ko

GOLD = pathlib.Path(__file__).resolve().parent / "golden"


def _t(d, name):
    return torch.from_numpy(np.asarray(d[name]))


def _rel(x, ref):
    x, ref = x.detach(), ref.detach()
    return float((x - ref).abs().max() / ref.abs().max().clamp_min(1e-30))


@pytest.mark.parametrize("variant", ["iso", "diag"])
def test_config0_forward_matches_reference(variant):
    d = np.load(GOLD / f"{variant}_config0_fp32.npz")
    q, k, v, alpha, omega, r = (_t(d, n) for n in ("q", "k", "v", "alpha", "omega", "r"))
    fn = ko.iso_recurrent if variant == "iso" else ko.diag_recurrent
    o, (S, prec) = fn(q, k, v, alpha, omega, r, output_final_state=True)
    assert _rel(o, _t(d, "o")) < 1e-5
    assert _rel(S, _t(d, "S")) < 1e-5
    assert _rel(prec, _t(d, "precision")) < 1e-5
    gfn = ko.iso_gain_tokenwise if variant == "iso" else ko.diag_gain_tokenwise
    gain, _ = gfn(k, alpha, omega, r)
    assert _rel(gain, _t(d, "gain")) < 1e-6


@pytest.mark.parametrize("variant", ["iso", "diag"])
@pytest.mark.parametrize("case", [0, 1])
def test_tiny_fp64_forward_and_grads_match_reference(variant, case):
    d = np.load(GOLD / f"{variant}_tiny{case}_fp64.npz")
    names = ["q", "k", "v", "alpha", "omega", "r", "initial_precision"]
    leaves = [_t(d, n).clone().requires_grad_(True) for n in names]
    has_mem = "initial_memory" in d.files
    mem = _t(d, "initial_memory").clone().requires_grad_(True) if has_mem else None
    info = float(d["info_scale"])
    sc = float(d["scale"])
    fn = ko.iso_recurrent if variant == "iso" else ko.diag_recurrent
    o, (S, prec) = fn(*leaves[:6], info_scale=None if np.isnan(info) else info,
                      scale=None if np.isnan(sc) else sc, initial_state=mem,
                      initial_precision=leaves[6], output_final_state=True)
    assert _rel(o, _t(d, "o")) < 1e-12
    assert _rel(S, _t(d, "S")) < 1e-12
    assert _rel(prec, _t(d, "precision")) < 1e-12
    loss = (o * _t(d, "w_o")).sum() + (S * _t(d, "w_S")).sum() + (prec * _t(d, "w_precision")).sum()
    grads = torch.autograd.grad(loss, leaves + ([mem] if has_mem else []))
    for n, g in zip(names + (["initial_memory"] if has_mem else []), grads):
        assert _rel(g, _t(d, f"d_{n}")) < 1e-10, n
