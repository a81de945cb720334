"""Diagonal KDN operators on MI355X: q/k normalisation, retention frontend, vector Kalman
gain, chunked memory scan.

Drop-in for the hot-path entry points of the reference module
``lit_gpt/kdn_ops/diag_kdn_chunk.py`` (ngocbh/kalman-delta-networks):

* ``_diag_kdn_normalize``                  (reference :2162-2168)
* ``_diag_kdn_frontend_precumsum_paired``  (reference :2471-2495)
* ``_diag_kdn_gain``                       (reference :2737-2791)
* ``chunk_kalman``                         (reference :3315-3329)

with the same argument order, dtypes, return values, autograd structure and Python errors.
State-carry extensions (keyword-only, default off): ``_diag_kdn_gain`` accepts a [B,H,K]
``initial_precision`` and ``output_final_state``; ``chunk_kalman`` accepts ``initial_state``
and ``output_final_state`` (semantics of the reference oracle,
diag_kdn_naive.py:503-567).  All arithmetic runs in ``libkdn_hip.so``; no fallback.

The paired ``g_cumsum`` uses the scan's 64-token chunk (the reference pairs 32); producer
and consumer are both in this module, so the pairing contract is unchanged: the scan's
backward returns a natural-log cotangent that the frontend reverse-sums per chunk.
"""
from __future__ import annotations

import math

import torch
from torch.autograd.function import once_differentiable

from . import _lib, _memscan

_DIAG_KDN_MEMORY_CHUNK_SIZE = 64
_DIAG_KDN_VECTOR_DTYPE = torch.bfloat16
_DIAG_KDN_STATE_DTYPE = torch.float32


# ---------------------------------------------------------------------------
# q/k normalisation
# ---------------------------------------------------------------------------

def _validate_diag_kdn_norm_inputs(q_raw, k_raw):
    """Reference diag_kdn_chunk.py:2025-2042."""
    for name, value in (("q_raw", q_raw), ("k_raw", k_raw)):
        if not isinstance(value, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if value.ndim != 4:
            raise ValueError(f"{name} must have rank 4 [B,T,H,K]")
        if not value.is_cuda:
            raise ValueError(f"{name} must be a GPU tensor")
        if value.dtype not in (torch.bfloat16, torch.float32):
            raise TypeError(f"{name} must be BF16 or FP32")
        if not value.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if q_raw.shape != k_raw.shape or q_raw.device != k_raw.device:
        raise ValueError("q_raw and k_raw must have matching shape and device")
    if q_raw.dtype != k_raw.dtype or q_raw.requires_grad != k_raw.requires_grad:
        raise ValueError("q_raw and k_raw must have matching dtype and grad mode")
    if q_raw.shape[-1] not in (64, 128):
        raise ValueError("q_raw and k_raw require K in {64,128}")


class _DiagKdnNormFunction(torch.autograd.Function):
    """Reference diag_kdn_chunk.py:2045-2076."""

    @staticmethod
    def forward(ctx, q_raw, k_raw):
        rows = q_raw.numel() // q_raw.shape[-1]
        K = q_raw.shape[-1]
        dev = q_raw.device
        q_memory = torch.empty(q_raw.shape, device=dev, dtype=torch.bfloat16)
        k_gain = torch.empty(q_raw.shape, device=dev, dtype=torch.float32)
        k_memory = torch.empty(q_raw.shape, device=dev, dtype=torch.bfloat16)
        q_norm = torch.empty(q_raw.shape[:-1], device=dev, dtype=torch.float32)
        k_norm = torch.empty_like(q_norm)
        with torch.cuda.device(dev):
            _lib.call("kdn_diag_norm_fwd", _lib.ptr(q_raw), _lib.ptr(k_raw), _lib.is_bf16(q_raw), rows, K,
                      _lib.ptr(q_memory), _lib.ptr(k_gain), _lib.ptr(k_memory), _lib.ptr(q_norm),
                      _lib.ptr(k_norm), _lib.stream_of(q_raw))
        ctx.save_for_backward(q_raw, k_raw, q_norm, k_norm)
        ctx.set_materialize_grads(False)
        return q_memory, k_gain, k_memory

    @staticmethod
    @once_differentiable
    def backward(ctx, d_q_memory, d_k_gain, d_k_memory):
        if not ctx.needs_input_grad[0]:
            d_q_memory = None
        if not ctx.needs_input_grad[1]:
            d_k_gain = None
            d_k_memory = None
        if d_q_memory is None and d_k_gain is None and d_k_memory is None:
            return None, None
        q_raw, k_raw, q_norm, k_norm = ctx.saved_tensors
        rows = q_raw.numel() // q_raw.shape[-1]
        d_q_memory = d_q_memory.to(torch.bfloat16).contiguous() if d_q_memory is not None else None
        d_k_gain = d_k_gain.float().contiguous() if d_k_gain is not None else None
        d_k_memory = d_k_memory.to(torch.bfloat16).contiguous() if d_k_memory is not None else None
        dq = torch.empty_like(q_raw) if d_q_memory is not None else None
        dk = torch.empty_like(k_raw) if (d_k_gain is not None or d_k_memory is not None) else None
        with torch.cuda.device(q_raw.device):
            _lib.call("kdn_diag_norm_bwd", _lib.ptr(q_raw), _lib.ptr(k_raw), _lib.is_bf16(q_raw), _lib.ptr(q_norm),
                      _lib.ptr(k_norm), _lib.ptr(d_q_memory), _lib.ptr(d_k_gain), _lib.ptr(d_k_memory), rows,
                      q_raw.shape[-1], _lib.ptr(dq), _lib.ptr(dk), _lib.stream_of(q_raw))
        return dq, dk


def _diag_kdn_normalize(q_raw, k_raw):
    """q/k -> (q_memory bf16, k_gain fp32, k_memory bf16), x / max(||x||, 1e-12) per row."""
    _validate_diag_kdn_norm_inputs(q_raw, k_raw)
    return _DiagKdnNormFunction.apply(q_raw, k_raw)


# ---------------------------------------------------------------------------
# Retention / noise frontend
# ---------------------------------------------------------------------------

def _validate_diag_kdn_frontend_inputs(retention_raw, omega_raw, r_raw, A_log, dt_bias, initial_precision_param):
    """Reference diag_kdn_chunk.py:2171-2215."""
    tensors = {"retention_raw": retention_raw, "omega_raw": omega_raw, "r_raw": r_raw, "A_log": A_log,
               "dt_bias": dt_bias, "initial_precision_param": initial_precision_param}
    for name, value in tensors.items():
        if not isinstance(value, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if not value.is_cuda:
            raise ValueError(f"{name} must be a GPU tensor")
        if value.device != retention_raw.device:
            raise ValueError("all DiagKDN frontend inputs must share one GPU device")
        if not value.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if retention_raw.ndim != 4:
        raise ValueError("retention_raw must have rank 4 [B,T,H,K]")
    B, T, H, K = retention_raw.shape
    if min(B, T, H) <= 0 or K not in (64, 128):
        raise ValueError("DiagKDN frontend requires non-empty B/T/H and K in {64,128}")
    if omega_raw.shape != (B, T, H, K):
        raise ValueError("omega_raw must match retention_raw")
    if r_raw.shape != (B, T, H):
        raise ValueError("r_raw must have shape [B,T,H]")
    if A_log.shape != (H,) or initial_precision_param.shape != (H,):
        raise ValueError("A_log and initial_precision_param must have shape [H]")
    if dt_bias.shape != (H, K):
        raise ValueError("dt_bias must have shape [H,K]")
    for name in ("retention_raw", "omega_raw", "r_raw"):
        if tensors[name].dtype != _DIAG_KDN_VECTOR_DTYPE:
            raise TypeError(f"{name} must be torch.bfloat16")
    for name in ("A_log", "dt_bias", "initial_precision_param"):
        if tensors[name].dtype != _DIAG_KDN_STATE_DTYPE:
            raise TypeError(f"{name} must be torch.float32")
    return B, T, H, K


class _DiagKdnFrontendFunction(torch.autograd.Function):
    """Reference diag_kdn_chunk.py:2426-2468."""

    @staticmethod
    def forward(ctx, retention_raw, omega_raw, r_raw, A_log, dt_bias, initial_precision_param):
        B, T, H, K = retention_raw.shape
        dev = retention_raw.device
        g_cumsum = torch.empty((B, T, H, K), device=dev, dtype=torch.float32)
        alpha = torch.empty_like(g_cumsum)
        omega = torch.empty_like(g_cumsum)
        r = torch.empty((B, T, H), device=dev, dtype=torch.float32)
        mu = torch.empty((H,), device=dev, dtype=torch.float32)
        with torch.cuda.device(dev):
            _lib.call("kdn_diag_frontend_fwd", _lib.ptr(retention_raw), _lib.ptr(omega_raw), _lib.ptr(r_raw),
                      _lib.ptr(A_log), _lib.ptr(dt_bias), _lib.ptr(initial_precision_param), B, T, H, K,
                      _DIAG_KDN_MEMORY_CHUNK_SIZE, _lib.ptr(g_cumsum), _lib.ptr(alpha), _lib.ptr(omega),
                      _lib.ptr(r), _lib.ptr(mu), _lib.stream_of(retention_raw))
        ctx.save_for_backward(retention_raw, omega_raw, r_raw, A_log, dt_bias, initial_precision_param, alpha)
        ctx.set_materialize_grads(False)
        return g_cumsum, alpha, omega, r, mu

    @staticmethod
    @once_differentiable
    def backward(ctx, d_g_cumsum, d_alpha, d_omega, d_r, d_initial_precision):
        retention_raw, omega_raw, r_raw, A_log, dt_bias, mu_param, alpha = ctx.saved_tensors
        B, T, H, K = retention_raw.shape
        dev = retention_raw.device
        need_ret, need_omega, need_r, need_A, need_dt, need_mu = ctx.needs_input_grad
        f = lambda t: t.float().contiguous() if t is not None else None  # noqa: E731
        d_g_cumsum, d_alpha, d_omega, d_r, d_initial_precision = map(
            f, (d_g_cumsum, d_alpha, d_omega, d_r, d_initial_precision))
        has_decay = d_g_cumsum is not None or d_alpha is not None
        dret = torch.empty_like(retention_raw) if (need_ret and has_decay) else None
        domega = torch.empty_like(omega_raw) if (need_omega and d_omega is not None) else None
        dr = torch.empty_like(r_raw) if (need_r and d_r is not None) else None
        dA = torch.empty_like(A_log) if (need_A and has_decay) else None
        ddt = torch.empty_like(dt_bias) if (need_dt and has_decay) else None
        dmu = torch.empty_like(mu_param) if (need_mu and d_initial_precision is not None) else None
        ws_bytes = _lib.size("kdn_diag_frontend_bwd_workspace_size", B, T, H, K, _DIAG_KDN_MEMORY_CHUNK_SIZE)
        ws = torch.empty((ws_bytes,), device=dev, dtype=torch.uint8)
        with torch.cuda.device(dev):
            _lib.call("kdn_diag_frontend_bwd", _lib.ptr(retention_raw), _lib.ptr(omega_raw), _lib.ptr(r_raw),
                      _lib.ptr(A_log), _lib.ptr(dt_bias), _lib.ptr(mu_param), _lib.ptr(alpha),
                      _lib.ptr(d_g_cumsum), _lib.ptr(d_alpha), _lib.ptr(d_omega), _lib.ptr(d_r),
                      _lib.ptr(d_initial_precision), B, T, H, K, _DIAG_KDN_MEMORY_CHUNK_SIZE, _lib.ptr(dret),
                      _lib.ptr(domega), _lib.ptr(dr), _lib.ptr(dA), _lib.ptr(ddt), _lib.ptr(dmu), _lib.ptr(ws),
                      ws_bytes, _lib.stream_of(retention_raw))
        return dret, domega, dr, dA, ddt, dmu


def _diag_kdn_frontend_precumsum_paired(retention_raw, omega_raw, r_raw, A_log, dt_bias, initial_precision_param):
    """(g_cumsum, alpha, omega, r, initial_precision): alpha = exp(-e^A softplus(f + dt_bias)),
    g_cumsum = chunk-local base-2 prefix of log(max(alpha, 1e-6)), omega = softplus(z),
    r = 0.01 + softplus(y), mu = 0.1 + softplus(p) (reference :2471-2495, kernel :1866-1905)."""
    _validate_diag_kdn_frontend_inputs(retention_raw, omega_raw, r_raw, A_log, dt_bias, initial_precision_param)
    return _DiagKdnFrontendFunction.apply(retention_raw, omega_raw, r_raw, A_log, dt_bias, initial_precision_param)


# ---------------------------------------------------------------------------
# Vector Kalman gain
# ---------------------------------------------------------------------------

def _diag_kdn_gain_forward(k, alpha, omega, r, initial_precision, *, save_state, output_final_state):
    B, T, H, K = k.shape
    dev = k.device
    prec_mode = 0 if initial_precision.ndim == 1 else 1
    kappa = torch.empty((B, T, H, K), device=dev, dtype=torch.float32)
    p_prev = torch.empty_like(kappa) if save_state else None
    D = torch.empty((B, T, H), device=dev, dtype=torch.float32) if save_state else None
    fprec = torch.empty((B, H, K), device=dev, dtype=torch.float32) if (output_final_state or save_state) else None
    ws_bytes = _lib.size("kdn_diag_gain_workspace_size", B, T, H, K)
    ws = torch.empty((ws_bytes,), device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        _lib.call("kdn_diag_gain_fwd", _lib.ptr(k), _lib.ptr(alpha), _lib.ptr(omega), _lib.ptr(r),
                  _lib.ptr(initial_precision), prec_mode, B, T, H, K, float(K), _lib.ptr(kappa), _lib.ptr(p_prev),
                  _lib.ptr(D), _lib.ptr(fprec), _lib.ptr(ws), ws_bytes, _lib.stream_of(k))
    return kappa, p_prev, D, fprec


class _DiagKdnGainFunction(torch.autograd.Function):
    """Reference diag_kdn_chunk.py:2686-2734 (omega, r enter detached; their raw-logit VJPs
    are fused into the gain backward)."""

    @staticmethod
    def forward(ctx, k, alpha, omega, r, initial_precision, omega_raw, r_raw, output_final_state):
        kappa, p_prev, D, fprec = _diag_kdn_gain_forward(k, alpha, omega, r, initial_precision, save_state=True,
                                                         output_final_state=output_final_state)
        ctx.save_for_backward(k, alpha, omega, r, initial_precision, omega_raw, r_raw, p_prev, D, fprec)
        ctx.set_materialize_grads(False)
        if output_final_state:
            return kappa, fprec
        return kappa

    @staticmethod
    @once_differentiable
    def backward(ctx, dkappa, d_final_precision=None):
        k, alpha, omega, r, mu, omega_raw, r_raw, p_prev, D, fprec = ctx.saved_tensors
        B, T, H, K = k.shape
        dev = k.device
        needs = ctx.needs_input_grad
        prec_mode = 0 if mu.ndim == 1 else 1
        dkappa = torch.zeros_like(k) if dkappa is None else dkappa.float().contiguous()
        dfp = d_final_precision.float().contiguous() if d_final_precision is not None else None
        dk = torch.empty_like(k)
        dalpha = torch.empty_like(alpha)
        domega_raw = torch.empty_like(omega_raw)
        dr_raw = torch.empty_like(r_raw)
        dmu = torch.empty_like(mu) if needs[4] else None
        G = torch.empty((B, T, H), device=dev, dtype=torch.float32)
        ws_bytes = _lib.size("kdn_diag_gain_workspace_size", B, T, H, K)
        ws = torch.empty((ws_bytes,), device=dev, dtype=torch.uint8)
        with torch.cuda.device(dev):
            _lib.call("kdn_diag_gain_bwd", _lib.ptr(k), _lib.ptr(alpha), _lib.ptr(omega), _lib.ptr(r), _lib.ptr(mu),
                      prec_mode, _lib.ptr(dkappa), _lib.ptr(p_prev), _lib.ptr(D), _lib.ptr(fprec), _lib.ptr(dfp),
                      _lib.ptr(omega_raw), _lib.ptr(r_raw), B, T, H, K, float(K), _lib.ptr(dk), _lib.ptr(dalpha),
                      _lib.ptr(domega_raw), _lib.ptr(dr_raw), _lib.ptr(dmu), _lib.ptr(G), _lib.ptr(ws), ws_bytes,
                      _lib.stream_of(k))
        return (dk if needs[0] else None, dalpha if needs[1] else None, None, None, dmu,
                domega_raw if needs[5] else None, dr_raw if needs[6] else None, None)


def _diag_kdn_gain(k_gain, alpha, omega, r, initial_precision, omega_raw, r_raw, *, output_final_state=False):
    """FP32 diagonal gain kappa [B,T,H,K] with fused raw-logit VJPs (reference :2737-2791).

    p_hat = alpha^2 p + omega;  kappa = p_hat k / (r + sum_i p_hat_i k_i^2);
    p' = p_hat / (1 + K k^2 / r p_hat);  p_0 = 1 / initial_precision ([H] or [B,H,K]).
    With ``output_final_state`` returns ``(kappa, final_precision [B,H,K])``.
    """
    tensors = {"k_gain": k_gain, "alpha": alpha, "omega": omega, "r": r, "initial_precision": initial_precision,
               "omega_raw": omega_raw, "r_raw": r_raw}
    for name, value in tensors.items():
        if not isinstance(value, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if not value.is_cuda:
            raise ValueError(f"{name} must be a GPU tensor")
        if value.device != k_gain.device:
            raise ValueError("all DiagKDN gain inputs must share one GPU device")
        if not value.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if k_gain.ndim != 4:
        raise ValueError("k_gain must have rank 4 [B,T,H,K]")
    B, T, H, K = k_gain.shape
    if min(B, T, H) <= 0 or K not in (64, 128):
        raise ValueError("DiagKDN gain requires non-empty B/T/H and K in {64,128}")
    expected = (B, T, H, K)
    for name in ("alpha", "omega", "omega_raw"):
        if tensors[name].shape != expected:
            raise ValueError(f"{name} must have shape {expected}")
    if r.shape != (B, T, H) or r_raw.shape != (B, T, H):
        raise ValueError("r and r_raw must have shape [B,T,H]")
    if initial_precision.shape not in ((H,), (B, H, K)):
        raise ValueError(f"initial_precision must have shape [{H}] or [{B},{H},{K}]")
    for name in ("k_gain", "alpha", "omega", "r", "initial_precision"):
        if tensors[name].dtype != torch.float32:
            raise TypeError(f"{name} must be torch.float32")
    if omega_raw.dtype != _DIAG_KDN_VECTOR_DTYPE or r_raw.dtype != _DIAG_KDN_VECTOR_DTYPE:
        raise TypeError("omega_raw and r_raw must be torch.bfloat16")
    if not (torch.is_grad_enabled() and any(t.requires_grad for t in (k_gain, alpha, initial_precision, omega_raw,
                                                                       r_raw))):
        # forward only: the backward's per-token state (p_prev, D) is not written
        kappa, _, _, fprec = _diag_kdn_gain_forward(k_gain, alpha, omega, r, initial_precision, save_state=False,
                                                    output_final_state=output_final_state)
        return (kappa, fprec) if output_final_state else kappa
    return _DiagKdnGainFunction.apply(k_gain, alpha, omega.detach(), r.detach(), initial_precision, omega_raw, r_raw,
                                      bool(output_final_state))


# ---------------------------------------------------------------------------
# Fused front half of the layer composition
# ---------------------------------------------------------------------------

_FRONT_MAX_ELEMS = 1 << 30  # one batch row of [T,H,K] per launch (the kernels' 32-bit offsets)


class _DiagKdnFrontFunction(torch.autograd.Function):
    """The layer's normalisation -> frontend -> gain chain (reference lit_gpt/diag_kdn.py:315-345 over
    diag_kdn_chunk.py:2162-2168, 2471-2495, 2737-2791) as one op.  Returns (q_memory, k_memory,
    g_cumsum, kappa, final_precision); alpha, omega, r and the fp32 gain key exist only inside the
    kernels, and the backward replays the precision per 16-token tile instead of reading p_prev."""

    @staticmethod
    def forward(ctx, q_raw, k_raw, retention_raw, omega_raw, r_raw, A_log, dt_bias, mu_param, initial_precision,
                save):
        B, T, H, K = q_raw.shape
        dev = q_raw.device
        rows = B * T * H
        q_memory = torch.empty((B, T, H, K), device=dev, dtype=torch.bfloat16)
        k_memory = torch.empty_like(q_memory)
        q_norm = torch.empty((B, T, H), device=dev, dtype=torch.float32)
        k_norm = torch.empty_like(q_norm)
        g_cumsum = torch.empty((B, T, H, K), device=dev, dtype=torch.float32)
        kappa = torch.empty_like(g_cumsum)
        fprec = torch.empty((B, H, K), device=dev, dtype=torch.float32)
        saved = (torch.empty((_lib.size("kdn_diag_front_saved_size", B, T, H, K) // 4,), device=dev,
                             dtype=torch.float32) if save else None)
        ws_bytes = _lib.size("kdn_diag_front_workspace_size", B, T, H, K)
        ws = torch.empty((ws_bytes,), device=dev, dtype=torch.uint8)
        prec_mode = 0 if initial_precision is None or initial_precision.ndim == 1 else 1
        with torch.cuda.device(dev):
            stream = _lib.stream_of(q_raw)
            _lib.call("kdn_diag_norm_fwd", _lib.ptr(q_raw), _lib.ptr(k_raw), _lib.is_bf16(q_raw), rows, K,
                      _lib.ptr(q_memory), None, _lib.ptr(k_memory), _lib.ptr(q_norm), _lib.ptr(k_norm), stream,
                      tag="diag_front_norm_fwd")
            _lib.call("kdn_diag_front_fwd", _lib.ptr(k_raw), _lib.is_bf16(k_raw), _lib.ptr(k_norm),
                      _lib.ptr(retention_raw), _lib.ptr(omega_raw), _lib.ptr(r_raw), _lib.ptr(A_log),
                      _lib.ptr(dt_bias), _lib.ptr(mu_param) if initial_precision is None else None,
                      _lib.ptr(initial_precision), prec_mode, B, T, H, K, _DIAG_KDN_MEMORY_CHUNK_SIZE, float(K),
                      _lib.ptr(g_cumsum), _lib.ptr(kappa), _lib.ptr(fprec), _lib.ptr(saved), _lib.ptr(ws), ws_bytes,
                      stream)
        if save:
            ctx.save_for_backward(q_raw, k_raw, q_norm, k_norm, retention_raw, omega_raw, r_raw, A_log, dt_bias,
                                  mu_param, initial_precision, saved, fprec)
        ctx.set_materialize_grads(False)
        return q_memory, k_memory, g_cumsum, kappa, fprec

    @staticmethod
    @once_differentiable
    def backward(ctx, d_q_memory, d_k_memory, d_g_cumsum, d_kappa, d_final_precision):
        (q_raw, k_raw, q_norm, k_norm, retention_raw, omega_raw, r_raw, A_log, dt_bias, mu_param, initial_precision,
         saved, fprec) = ctx.saved_tensors
        B, T, H, K = q_raw.shape
        dev = q_raw.device
        needs = ctx.needs_input_grad
        prec_mode = 0 if initial_precision is None or initial_precision.ndim == 1 else 1
        d_g_cumsum = (torch.zeros((B, T, H, K), device=dev, dtype=torch.float32) if d_g_cumsum is None
                      else d_g_cumsum.float().contiguous())
        d_kappa = (torch.zeros((B, T, H, K), device=dev, dtype=torch.float32) if d_kappa is None
                   else d_kappa.float().contiguous())
        d_k_memory = d_k_memory.to(torch.bfloat16).contiguous() if d_k_memory is not None else None
        dfp = d_final_precision.float().contiguous() if d_final_precision is not None else None
        dk = torch.empty_like(k_raw) if needs[1] else None
        dret = torch.empty_like(retention_raw)
        domega = torch.empty_like(omega_raw)
        dr = torch.empty_like(r_raw)
        dA = torch.empty_like(A_log) if needs[5] else None
        ddt = torch.empty_like(dt_bias) if needs[6] else None
        dmu = torch.empty_like(mu_param) if (needs[7] and initial_precision is None) else None
        dinit = torch.empty_like(initial_precision) if (initial_precision is not None and needs[8]) else None
        ws_bytes = _lib.size("kdn_diag_front_workspace_size", B, T, H, K)
        ws = torch.empty((ws_bytes,), device=dev, dtype=torch.uint8)
        dq = None
        with torch.cuda.device(dev):
            stream = _lib.stream_of(q_raw)
            _lib.call("kdn_diag_front_bwd", _lib.ptr(k_raw), _lib.is_bf16(k_raw), _lib.ptr(k_norm),
                      _lib.ptr(retention_raw), _lib.ptr(omega_raw), _lib.ptr(r_raw), _lib.ptr(A_log),
                      _lib.ptr(dt_bias), _lib.ptr(mu_param) if initial_precision is None else None,
                      _lib.ptr(initial_precision), prec_mode, _lib.ptr(saved), _lib.ptr(fprec), _lib.ptr(d_g_cumsum),
                      _lib.ptr(d_kappa), _lib.ptr(d_k_memory), _lib.ptr(dfp), B, T, H, K,
                      _DIAG_KDN_MEMORY_CHUNK_SIZE, float(K), _lib.ptr(dk), _lib.ptr(dret), _lib.ptr(domega),
                      _lib.ptr(dr), _lib.ptr(dA), _lib.ptr(ddt), _lib.ptr(dmu), _lib.ptr(dinit), _lib.ptr(ws),
                      ws_bytes, stream)
            if needs[0] and d_q_memory is not None:
                dq = torch.empty_like(q_raw)
                d_q_memory = d_q_memory.to(torch.bfloat16).contiguous()
                _lib.call("kdn_diag_norm_bwd", _lib.ptr(q_raw), _lib.ptr(k_raw), _lib.is_bf16(q_raw),
                          _lib.ptr(q_norm), _lib.ptr(k_norm), _lib.ptr(d_q_memory), None, None, B * T * H, K,
                          _lib.ptr(dq), None, stream, tag="diag_front_norm_bwd")
        return (dq, dk, dret if needs[2] else None, domega if needs[3] else None, dr if needs[4] else None, dA, ddt,
                dmu, dinit, None)


def diag_kdn_front(q_raw, k_raw, retention_raw, omega_raw, r_raw, A_log, dt_bias, initial_precision_param, *,
                   initial_precision=None, output_final_state=False):
    """``_diag_kdn_normalize`` -> ``_diag_kdn_frontend_precumsum_paired`` -> ``_diag_kdn_gain`` as the
    layer composes them (reference lit_gpt/diag_kdn.py:315-345), fused: returns
    ``(q_memory, k_memory, g_cumsum, kappa)`` (plus ``final_precision`` [B,H,K] with
    ``output_final_state``), equal to the three ops' outputs.  The prior precision is the frontend's
    ``0.1 + softplus(initial_precision_param)`` unless ``initial_precision`` ([H] or [B,H,K]) is given.
    Same argument checks and errors as the three ops."""
    _validate_diag_kdn_norm_inputs(q_raw, k_raw)
    B, T, H, K = _validate_diag_kdn_frontend_inputs(retention_raw, omega_raw, r_raw, A_log, dt_bias,
                                                    initial_precision_param)
    if tuple(q_raw.shape) != (B, T, H, K) or q_raw.device != retention_raw.device:
        raise ValueError("q_raw and k_raw must match retention_raw's shape and device")
    if initial_precision is not None:
        if not isinstance(initial_precision, torch.Tensor):
            raise TypeError("initial_precision must be a torch.Tensor")
        if initial_precision.shape not in ((H,), (B, H, K)):
            raise ValueError(f"initial_precision must have shape [{H}] or [{B},{H},{K}]")
        if initial_precision.dtype != torch.float32:
            raise TypeError("initial_precision must be torch.float32")
        if not initial_precision.is_contiguous() or initial_precision.device != retention_raw.device:
            raise ValueError("initial_precision must be a contiguous tensor on the inputs' device")
    if T * H * K > _FRONT_MAX_ELEMS:  # longer than the fused kernels address: the three ops, still all HIP
        q_memory, k_gain, k_memory = _diag_kdn_normalize(q_raw, k_raw)
        g_cumsum, alpha, omega, r, mu = _diag_kdn_frontend_precumsum_paired(
            retention_raw, omega_raw, r_raw, A_log, dt_bias, initial_precision_param)
        prec = mu if initial_precision is None else initial_precision
        out = _diag_kdn_gain(k_gain, alpha, omega, r, prec, omega_raw, r_raw, output_final_state=output_final_state)
        if output_final_state:
            return q_memory, k_memory, g_cumsum, out[0], out[1]
        return q_memory, k_memory, g_cumsum, out
    inputs = (q_raw, k_raw, retention_raw, omega_raw, r_raw, A_log, dt_bias, initial_precision_param,
              initial_precision)
    save = torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in inputs)
    q_memory, k_memory, g_cumsum, kappa, fprec = _DiagKdnFrontFunction.apply(*inputs, save)
    if output_final_state:
        return q_memory, k_memory, g_cumsum, kappa, fprec
    return q_memory, k_memory, g_cumsum, kappa


# ---------------------------------------------------------------------------
# Chunked memory scan
# ---------------------------------------------------------------------------

def _validate_diag_kdn_memory_inputs(q, k, kappa, v, g_cumsum, scale):
    """Reference diag_kdn_chunk.py:2794-2821."""
    tensors = {"q": q, "k": k, "kappa": kappa, "v": v, "g_cumsum": g_cumsum}
    for name, value in tensors.items():
        if not isinstance(value, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if value.ndim != 4:
            raise ValueError(f"{name} must have rank 4 [B,T,H,D]")
        if not value.is_cuda:
            raise ValueError(f"{name} must be a GPU tensor")
        if value.device != q.device:
            raise ValueError("all DiagKDN memory inputs must share one GPU device")
        if not value.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    B, T, H, K = q.shape
    if min(B, T, H) <= 0 or K not in (64, 128):
        raise ValueError("DiagKDN memory requires non-empty B/T/H and K in {64,128}")
    expected = (B, T, H, K)
    for name in ("k", "kappa", "v", "g_cumsum"):
        if tensors[name].shape != expected:
            raise ValueError(f"{name} must have shape {expected}")
    for name in ("q", "k", "v"):
        if tensors[name].dtype != _DIAG_KDN_VECTOR_DTYPE:
            raise TypeError(f"{name} must be torch.bfloat16")
    if kappa.dtype != _DIAG_KDN_STATE_DTYPE or g_cumsum.dtype != _DIAG_KDN_STATE_DTYPE:
        raise TypeError("kappa and g_cumsum must be torch.float32")
    if type(scale) is not float or not math.isfinite(scale):
        raise TypeError("scale must be an exact finite float")
    return B, T, H, K


class _DiagKdnMemoryFunction(torch.autograd.Function):
    """Reference diag_kdn_chunk.py:3247-3312 (fp32 output; fp32 output cotangent).

    ``out_dtype`` bf16 is the layer composition's ``chunk_kalman(...).to(v.dtype)``
    (diag_kdn.py:342-345) done in the kernel: the fp32 accumulator is rounded to bf16 at the
    store, and the bf16 cotangent is the cast's exact upcast, so results are identical."""

    @staticmethod
    def forward(ctx, q, k, kappa, v, g_cumsum, scale, initial_state, output_final_state, out_dtype=torch.float32):
        # no input needs a gradient (inference), or the "recompute" backward mode: the intermediates
        # only the backward reads are skipped (in that mode the backward rebuilds them from the inputs)
        need_backward = any(ctx.needs_input_grad)
        ctx.recompute = need_backward and _memscan.backward_mode() == "recompute"
        with torch.cuda.device(q.device):
            o, saved, ht = _memscan.mem_fwd(q, k, kappa, False, v, g_cumsum, scale, initial_state=initial_state,
                                            output_final_state=output_final_state, out_dtype=out_dtype,
                                            need_backward=need_backward and not ctx.recompute)
        if need_backward:
            ctx.save_for_backward(q, k, kappa, v, g_cumsum, None if ctx.recompute else saved,
                                  initial_state if ctx.recompute else None)
        ctx.scale = scale
        ctx.has_h0 = initial_state is not None
        ctx.set_materialize_grads(False)
        if output_final_state:
            return o, ht
        return o

    @staticmethod
    @once_differentiable
    def backward(ctx, do, d_final_state=None):
        q, k, kappa, v, g_cumsum, saved, h0 = ctx.saved_tensors
        if do is None and d_final_state is None:
            return None, None, None, None, None, None, None, None, None
        B, T, H, K = q.shape
        V = v.shape[-1]
        dev = q.device
        if do is None:
            do = torch.zeros((B, T, H, V), device=dev, dtype=torch.float32)
        elif do.dtype not in (torch.bfloat16, torch.float32):
            do = do.float().contiguous()
        else:
            do = do.contiguous()
        need_h0 = ctx.has_h0 and ctx.needs_input_grad[6]
        with torch.cuda.device(dev):
            if ctx.recompute:
                saved = _memscan.rebuild_saved(q, k, kappa, False, v, g_cumsum, ctx.scale, initial_state=h0)
            dq, dk, dv, dkappa, dg, dh0 = _memscan.mem_bwd(q, k, kappa, False, v, g_cumsum, saved, ctx.scale, do,
                                                          d_final_state=d_final_state,
                                                          need_initial_state_grad=need_h0)
        return dq, dk, dkappa, dv, dg, None, dh0, None, None


def chunk_kalman(q_memory, k_memory, kappa, v, g_cumsum, scale, *, initial_state=None, output_final_state=False):
    """Diagonal KDN memory scan o [B,T,H,V] fp32 (reference :3315-3329).

    With ``output_final_state`` returns ``(o, final_state [B,H,K,V] fp32)``; ``initial_state``
    [B,H,K,V] fp32 seeds the memory (reference oracle initial_memory).
    """
    B, T, H, K = _validate_diag_kdn_memory_inputs(q_memory, k_memory, kappa, v, g_cumsum, scale)
    if initial_state is not None:
        if initial_state.shape != (B, H, K, v.shape[-1]) or not initial_state.is_cuda:
            raise ValueError(f"initial_state must be a GPU tensor of shape {(B, H, K, v.shape[-1])}")
        if initial_state.device != q_memory.device:
            raise ValueError("initial_state must be on the same device as q")
    return _DiagKdnMemoryFunction.apply(q_memory, k_memory, kappa, v, g_cumsum, scale, initial_state,
                                        bool(output_final_state))


def _chunk_kalman_as(q_memory, k_memory, kappa, v, g_cumsum, scale, *, initial_state=None,
                     output_final_state=False, out_dtype=torch.bfloat16):
    """``chunk_kalman(...)`` followed by ``.to(out_dtype)``, with the cast done at the kernel's store
    (the layer composition of diag_kdn.py:342-345); same validation and results."""
    B, T, H, K = _validate_diag_kdn_memory_inputs(q_memory, k_memory, kappa, v, g_cumsum, scale)
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("out_dtype must be torch.bfloat16 or torch.float32")
    if initial_state is not None:
        if initial_state.shape != (B, H, K, v.shape[-1]) or not initial_state.is_cuda:
            raise ValueError(f"initial_state must be a GPU tensor of shape {(B, H, K, v.shape[-1])}")
        if initial_state.device != q_memory.device:
            raise ValueError("initial_state must be on the same device as q")
    return _DiagKdnMemoryFunction.apply(q_memory, k_memory, kappa, v, g_cumsum, scale, initial_state,
                                        bool(output_final_state), out_dtype)


__all__ = ("chunk_kalman", "_diag_kdn_normalize", "_diag_kdn_frontend_precumsum_paired", "_diag_kdn_gain")
