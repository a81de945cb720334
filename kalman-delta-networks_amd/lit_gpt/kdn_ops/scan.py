"""The KDN mixer scan: the kdn_ops calls of one layer, composed as the reference layers do.

``iso_kdn_scan`` follows lit_gpt/iso_kdn.py:277-304 (gate frontend -> scalar gain ->
chunked memory scan with in-op q/k normalisation), with the first two as one fused op
(``iso_kdn_front``); ``diag_kdn_scan`` follows
lit_gpt/diag_kdn.py:315-345 (q/k normalisation -> frontend -> vector gain -> memory scan,
output materialised at v's dtype), with the first three as one fused op (``diag_kdn_front``).  Projections, short convolutions and the gated output
norm of the layers are not part of the scan.
"""
from __future__ import annotations

from .diag_kdn_chunk import _chunk_kalman_as, diag_kdn_front
from .iso_kdn_chunk import _chunk_kda_precumsum_paired, iso_kdn_front


def iso_kdn_scan(q, k, v, g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias, initial_precision_param,
                 *, omega_min: float = 0.0, r_min: float = 0.01, info_scale: float | None = None):
    """q, k, v, g_raw [B,T,H,d]; omega_r_raw [B,T,2H]; dt_bias [H*K]; returns o [B,T,H,V]."""
    K = q.shape[-1]
    # gate -> gain as one fused op (same results as the two reference ops)
    g_cumsum, beta = iso_kdn_front(g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias, initial_precision_param,
                                   omega_min, r_min, head_dim=K, info_scale=float(K) if info_scale is None else info_scale)
    return _chunk_kda_precumsum_paired(q=q, k=k, v=v, g_cumsum=g_cumsum, beta=beta)


def diag_kdn_scan(q, k, v, retention_raw, omega_raw, r_raw, A_log, dt_bias, initial_precision_param,
                  *, initial_state=None, initial_precision=None, output_final_state: bool = False):
    """q, k, v, retention_raw, omega_raw [B,T,H,d] bf16; r_raw [B,T,H]; dt_bias [H,K];
    returns o [B,T,H,V] in v's dtype.

    Long-context continuation (the reference oracle's initial_memory / initial_precision,
    diag_kdn_naive.py:503-516): ``initial_state`` [B,H,K,V] fp32 seeds the memory,
    ``initial_precision`` [B,H,K] fp32 replaces the learned [H] prior, and with
    ``output_final_state`` the call returns ``(o, (final_state, final_precision))``."""
    K = q.shape[-1]
    # normalisation -> frontend -> gain as one fused op (same results as the three reference ops)
    front = diag_kdn_front(q, k, retention_raw, omega_raw, r_raw, A_log, dt_bias, initial_precision_param,
                           initial_precision=initial_precision, output_final_state=output_final_state)
    q_memory, k_memory, g_cumsum, kappa = front[:4]
    scale = float(K ** -0.5)
    if output_final_state:
        out, final_state = _chunk_kalman_as(q_memory, k_memory, kappa, v, g_cumsum, scale,
                                            initial_state=initial_state, output_final_state=True, out_dtype=v.dtype)
        return out, (final_state, front[4])
    # chunk_kalman(...).to(v.dtype) with the cast at the kernel's store
    return _chunk_kalman_as(q_memory, k_memory, kappa, v, g_cumsum, scale, initial_state=initial_state,
                            out_dtype=v.dtype)
