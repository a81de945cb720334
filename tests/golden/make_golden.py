"""Write golden vectors from the reference's own PyTorch recurrence oracles.

Run in the build container only (``/root/reference`` does not exist on the GPU
box):  ``python tests/golden/make_golden.py``.  It loads
``lit_gpt/kdn_ops/iso_kdn_naive.py`` and ``diag_kdn_naive.py`` by file path (the
package ``lit_gpt/__init__.py`` imports flash-attn/lightning, which are absent),
calls the public tokenwise oracles

  * ``iso_kdn_gain_naive``       (iso_kdn_naive.py:200-251)
  * ``naive_recurrent_iso_kdn``  (iso_kdn_naive.py:376-440)
  * ``diag_kdn_gain_naive``      (diag_kdn_naive.py:217-276)
  * ``naive_recurrent_diag_kdn`` (diag_kdn_naive.py:503-567)

on seeded inputs, and stores inputs, outputs and autograd gradients as
``.npz`` data files next to this script.  Nothing from the reference is stored
except these numeric vectors.
"""
from __future__ import annotations

import importlib.util
import pathlib

import numpy as np
import torch
import torch.nn.functional as F

REF = pathlib.Path("/root/reference/lit_gpt/kdn_ops")
OUT = pathlib.Path(__file__).resolve().parent


def _load(name: str):
    spec = importlib.util.spec_from_file_location(f"_ref_{name}", REF / f"{name}.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _inputs(gen, B, T, H, K, V, *, diag: bool, dtype):
    """Draw order q, k, v, alpha_pre, omega_pre, r_pre (config-0 distributions)."""
    q = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64)
    k = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64)
    v = torch.randn(B, T, H, V, generator=gen, dtype=torch.float64)
    alpha = torch.sigmoid(2.0 + 0.5 * torch.randn(B, T, H, K, generator=gen, dtype=torch.float64))
    wshape = (B, T, H, K) if diag else (B, T, H)
    omega = F.softplus(torch.randn(*wshape, generator=gen, dtype=torch.float64))
    r = 0.01 + F.softplus(torch.randn(B, T, H, generator=gen, dtype=torch.float64))
    q = q / q.norm(dim=-1, keepdim=True)
    k = k / k.norm(dim=-1, keepdim=True)
    return [x.to(dtype) for x in (q, k, v, alpha, omega, r)]


def _np(x):
    return x.detach().cpu().numpy()


def config0(iso, diag):
    """BASELINE config 0 shape (B=1, H=2, T=256, d=64), fp32, forward only, seed 0."""
    for variant, mod in (("iso", iso), ("diag", diag)):
        gen = torch.Generator().manual_seed(0)
        q, k, v, alpha, omega, r = _inputs(gen, 1, 256, 2, 64, 64, diag=variant == "diag",
                                           dtype=torch.float32)
        fn = mod.naive_recurrent_iso_kdn if variant == "iso" else mod.naive_recurrent_diag_kdn
        gfn = mod.iso_kdn_gain_naive if variant == "iso" else mod.diag_kdn_gain_naive
        with torch.no_grad():
            o, (S, prec) = fn(q, k, v, alpha, omega, r, output_final_state=True)
            gain, _ = gfn(k, alpha, omega, r)
        np.savez_compressed(OUT / f"{variant}_config0_fp32.npz",
                            q=_np(q), k=_np(k), v=_np(v), alpha=_np(alpha), omega=_np(omega), r=_np(r),
                            o=_np(o), S=_np(S), precision=_np(prec), gain=_np(gain))


def tiny_fp64_grads(iso, diag):
    """Small fp64 cases exercising every optional argument, with autograd gradients."""
    cases = [
        dict(B=2, T=19, H=2, K=8, V=6, info_scale=3.0, scale=0.7, init_prec="BH", init_mem=True),
        dict(B=1, T=7, H=3, K=4, V=5, info_scale=None, scale=None, init_prec="H", init_mem=False),
    ]
    for variant, mod in (("iso", iso), ("diag", diag)):
        fn = mod.naive_recurrent_iso_kdn if variant == "iso" else mod.naive_recurrent_diag_kdn
        for ci, c in enumerate(cases):
            gen = torch.Generator().manual_seed(100 + ci)
            B, T, H, K, V = c["B"], c["T"], c["H"], c["K"], c["V"]
            q, k, v, alpha, omega, r = _inputs(gen, B, T, H, K, V, diag=variant == "diag",
                                               dtype=torch.float64)
            # Unnormalised keys exercise |k|^2 != 1 in both gain recurrences.
            k = k * (0.5 + torch.rand(B, T, H, 1, generator=gen, dtype=torch.float64))
            if c["init_prec"] == "BH":
                if variant == "diag":
                    prec0 = 0.2 + torch.rand(B, H, K, generator=gen, dtype=torch.float64)
                else:
                    prec0 = 0.2 + torch.rand(B, H, generator=gen, dtype=torch.float64)
            else:
                prec0 = 0.2 + torch.rand(H, generator=gen, dtype=torch.float64)
            mem0 = (0.1 * torch.randn(B, H, K, V, generator=gen, dtype=torch.float64)
                    if c["init_mem"] else None)
            leaves = [x.clone().requires_grad_(True) for x in (q, k, v, alpha, omega, r, prec0)]
            mem_leaf = mem0.clone().requires_grad_(True) if mem0 is not None else None
            o, (S, prec) = fn(*leaves[:6], info_scale=c["info_scale"], scale=c["scale"],
                              initial_memory=mem_leaf, initial_precision=leaves[6],
                              output_final_state=True)
            wo = torch.randn(o.shape, generator=gen, dtype=torch.float64)
            wS = torch.randn(S.shape, generator=gen, dtype=torch.float64)
            wp = torch.randn(prec.shape, generator=gen, dtype=torch.float64)
            loss = (o * wo).sum() + (S * wS).sum() + (prec * wp).sum()
            grads = torch.autograd.grad(loss, leaves + ([mem_leaf] if mem_leaf is not None else []))
            names = ["q", "k", "v", "alpha", "omega", "r", "initial_precision"]
            if mem_leaf is not None:
                names.append("initial_memory")
            data = {n: _np(x) for n, x in zip(names[:7], leaves)}
            if mem_leaf is not None:
                data["initial_memory"] = _np(mem_leaf)
            data.update({f"d_{n}": _np(g) for n, g in zip(names, grads)})
            data.update(o=_np(o), S=_np(S), precision=_np(prec), w_o=_np(wo), w_S=_np(wS),
                        w_precision=_np(wp),
                        info_scale=np.array(np.nan if c["info_scale"] is None else c["info_scale"]),
                        scale=np.array(np.nan if c["scale"] is None else c["scale"]))
            np.savez_compressed(OUT / f"{variant}_tiny{ci}_fp64.npz", **data)


def main():
    torch.set_num_threads(4)
    iso = _load("iso_kdn_naive")
    diag = _load("diag_kdn_naive")
    config0(iso, diag)
    tiny_fp64_grads(iso, diag)
    for p in sorted(OUT.glob("*.npz")):
        print(p.name, p.stat().st_size)


if __name__ == "__main__":
    main()
