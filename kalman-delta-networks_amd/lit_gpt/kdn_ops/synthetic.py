"""Seeded synthetic inputs for the KDN mixer scan (benchmark and parity workloads).

Distributions (drawn in this order from one CPU generator): q, k ~ N(0,1); v ~ N(0,1);
per-channel retention alpha = sigmoid(N(2, 0.5)); process-noise pre-activation ~ N(0,1)
([B,T,H] for iso, [B,T,H,K] for diag) through softplus; observation noise
r = 0.01 + softplus(N(0,1)); initial precision 1; upstream gradient dO ~ N(0,1).

The scan consumes raw pre-activations, so alpha is produced through the layer's own
gate parameterisation with A_log = 0 and dt_bias = 0: g_raw = log(expm1(-log alpha)) gives
softplus(g_raw) = -log alpha exactly (before rounding to the input dtype).
"""
from __future__ import annotations

import math

import torch


def make_inputs(variant: str, B: int, T: int, H: int, K: int, *, seed: int = 0, device="cuda",
                dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=g)
    k = torch.randn(B, T, H, K, generator=g)
    v = torch.randn(B, T, H, K, generator=g)
    alpha = torch.sigmoid(2.0 + 0.5 * torch.randn(B, T, H, K, generator=g))
    g_raw = torch.log(torch.expm1(-torch.log(alpha)))
    if variant == "iso":
        omega_pre = torch.randn(B, T, H, generator=g)
    else:
        omega_pre = torch.randn(B, T, H, K, generator=g)
    r_pre = torch.randn(B, T, H, generator=g)
    do = torch.randn(B, T, H, K, generator=g)
    mu_param = torch.full((H,), math.log(math.expm1(1.0 - 0.1)))
    to = lambda x, dt=dtype: x.to(device=device, dtype=dt).contiguous()  # noqa: E731
    A_log = torch.zeros(H)
    if variant == "iso":
        orr = torch.cat([omega_pre, r_pre], dim=-1)
        return dict(q=to(q), k=to(k), v=to(v), g_raw=to(g_raw), omega_r_raw=to(orr),
                    omega_bias=to(torch.zeros(H), torch.float32), r_bias=to(torch.zeros(H), torch.float32),
                    A_log=to(A_log, torch.float32), dt_bias=to(torch.zeros(H * K), torch.float32),
                    initial_precision_param=to(mu_param, torch.float32)), to(do)
    return dict(q=to(q), k=to(k), v=to(v), retention_raw=to(g_raw), omega_raw=to(omega_pre), r_raw=to(r_pre),
                A_log=to(A_log, torch.float32), dt_bias=to(torch.zeros(H, K), torch.float32),
                initial_precision_param=to(mu_param, torch.float32)), to(do)


GRAD_KEYS = {
    "iso": ("q", "k", "v", "g_raw", "omega_r_raw", "omega_bias", "r_bias", "A_log", "dt_bias",
            "initial_precision_param"),
    "diag": ("q", "k", "v", "retention_raw", "omega_raw", "r_raw", "A_log", "dt_bias", "initial_precision_param"),
}
