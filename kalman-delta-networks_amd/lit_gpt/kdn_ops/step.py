"""One token of the KDN memory recurrence with a carried state (``kdn_mem_step``).

The reference runs KDN layers on fixed-length sequences only and refuses caching
(``lit_gpt/model.py:104,184``); its naive recurrences (``iso_kdn_naive.py:308-332``,
``diag_kdn_naive.py:479-500``) define what one step does:

    S_hat = exp2(g) (.) S;  delta = v - S_hat^T k;  S = S_hat + kappa delta^T;  o = scale S^T q

with ``g`` the token's base-2 log decay (the gate frontends' ``g_cumsum`` at T = 1).  The state
is the chunked scan's ``initial_state`` / ``final_state`` layout [B,H,K,V] fp32, so a prefill's
final state continues here token by token, and a state written here continues a later prefill.
"""
from __future__ import annotations

import torch

from . import _lib


def kdn_memory_step(q, k, v, g_cumsum, *, state, beta=None, kappa=None, scale=None, out_dtype=None):
    """Advance ``state`` [B,H,K,V] fp32 in place by one token and return o [B,1,H,V].

    q, k [B,1,H,K] and v [B,1,H,V] (bf16 or fp32; cast to q's dtype); ``g_cumsum`` [B,1,H,K]
    fp32 base-2 log decay.  Isotropic form: ``beta`` [B,1,H] fp32, q and k L2-normalised inside
    as the chunked scan does.  Diagonal form: ``kappa`` [B,1,H,K] fp32, q and k already
    normalised.  ``out_dtype`` defaults to q's dtype.
    """
    if (beta is None) == (kappa is None):
        raise ValueError("pass exactly one of beta (isotropic) or kappa (diagonal)")
    if q.ndim != 4 or q.shape[1] != 1 or k.shape != q.shape:
        raise ValueError(f"q and k must share shape [B,1,H,K], got {tuple(q.shape)} and {tuple(k.shape)}")
    B, _, H, K = q.shape
    if v.ndim != 4 or v.shape[:3] != (B, 1, H):
        raise ValueError(f"v must have shape [{B},1,{H},V], got {tuple(v.shape)}")
    V = v.shape[-1]
    if K not in (64, 128) or V not in (64, 128):
        raise ValueError(f"the step kernel supports K, V in {{64, 128}}, got K={K}, V={V}")
    if g_cumsum.shape != (B, 1, H, K) or g_cumsum.dtype != torch.float32:
        raise ValueError(f"g_cumsum must be fp32 [{B},1,{H},{K}], got {g_cumsum.dtype} {tuple(g_cumsum.shape)}")
    if state.shape != (B, H, K, V) or state.dtype != torch.float32 or not state.is_contiguous():
        raise ValueError(f"state must be a contiguous fp32 tensor of shape {(B, H, K, V)}")
    iso = beta is not None
    gate = beta if iso else kappa
    want = (B, 1, H) if iso else (B, 1, H, K)
    if gate.shape != want:
        raise ValueError(f"{'beta' if iso else 'kappa'} must have shape {want}, got {tuple(gate.shape)}")
    if q.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"q must be bf16 or fp32, got {q.dtype}")
    out_dtype = q.dtype if out_dtype is None else out_dtype
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"out_dtype must be bf16 or fp32, got {out_dtype}")
    _lib.require_device(q, k, v, g_cumsum, state, gate)
    dt = q.dtype
    q, k, v = (x.to(dt).contiguous() for x in (q, k, v))
    gate = gate.float().contiguous()
    g_cumsum = g_cumsum.contiguous()
    o = torch.empty((B, 1, H, V), device=q.device, dtype=out_dtype)
    scale = K ** -0.5 if scale is None else float(scale)
    with torch.cuda.device(q.device):
        _lib.call("kdn_mem_step", _lib.ptr(q), _lib.ptr(k), _lib.ptr(gate), int(iso), _lib.ptr(v),
                  _lib.is_bf16(q), _lib.ptr(g_cumsum), B, H, K, V, scale, _lib.ptr(state), _lib.ptr(o),
                  _lib.is_bf16(o), _lib.stream_of(q), tag="mem_step")
    return o


__all__ = ("kdn_memory_step",)
