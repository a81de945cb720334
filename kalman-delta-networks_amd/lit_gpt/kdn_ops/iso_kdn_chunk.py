"""Isotropic KDN operators on MI355X: gate frontend, scalar Kalman gain, chunked memory scan.

Drop-in for the hot-path entry points of the reference module
``lit_gpt/kdn_ops/iso_kdn_chunk.py`` (ngocbh/kalman-delta-networks):

* ``_iso_kdn_gate_precumsum_paired``  (reference :1395-1436)
* ``iso_kdn_gain``                    (reference :1965-2031)
* ``_chunk_kda_precumsum_paired``     (reference :2241-2285)
* ``qkv_causal_conv1d``               (reference :468-478; implemented in ``short_conv.py``)

with the same argument order, dtypes, return tuples, autograd.Function structure and
Python-side errors.  ``iso_kdn_front`` is the first two as the layer composes them, fused
(same results; no counterpart in the reference).  All arithmetic runs in the HIP library (``libkdn_hip.so``); there is
no PyTorch or CPU fallback.  The packed projections of the reference module (plain GEMMs,
iso_kdn_chunk.py:480-729) are not part of this package.
"""
from __future__ import annotations

import math
from numbers import Real

import torch

from . import _lib, _memscan
from .short_conv import qkv_causal_conv1d  # the reference module also defines it (:468-478)

ISO_GATE_CHUNK_SIZE = 64
KDA_CHUNK_SIZE = 64
_L2NORM_EPS = 1e-6


# ---------------------------------------------------------------------------
# Gate frontend
# ---------------------------------------------------------------------------

def _validate_iso_gate_inputs(g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias,
                              initial_precision_param, omega_min, r_min):
    """Reference iso_kdn_chunk.py:1012-1056."""
    if g_raw.ndim != 4:
        raise ValueError(f"g_raw must have shape [B,T,H,K], got {tuple(g_raw.shape)}")
    B, T, H, K = g_raw.shape
    if K == 0:
        raise ValueError("g_raw's K dimension must be nonzero")
    if omega_r_raw.shape != (B, T, 2 * H):
        raise ValueError(f"omega_r_raw must have shape {(B, T, 2 * H)}, got {tuple(omega_r_raw.shape)}")
    if omega_r_raw.stride(-1) != 1:
        raise ValueError(f"omega_r_raw's head dimension must be contiguous, got strides={omega_r_raw.stride()}")
    for name, value in (("omega_bias", omega_bias), ("r_bias", r_bias)):
        if value.shape != (H,):
            raise ValueError(f"{name} must have shape [{H}], got {tuple(value.shape)}")
    if A_log.shape != (H,):
        raise ValueError(f"A_log must have shape [{H}], got {tuple(A_log.shape)}")
    if dt_bias.shape != (H * K,):
        raise ValueError(f"dt_bias must have shape [{H * K}], got {tuple(dt_bias.shape)}")
    if initial_precision_param.shape != (H,):
        raise ValueError(
            f"initial_precision_param must have shape [{H}], got {tuple(initial_precision_param.shape)}")
    inputs = (g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias, initial_precision_param)
    if not all(value.is_cuda for value in inputs):
        raise ValueError("_iso_kdn_gate_precumsum_paired is a GPU-only HIP op")
    if any(value.device != g_raw.device for value in inputs[1:]):
        raise ValueError("all scalar-preparation inputs must be on the same GPU device")
    for name, value in (("g_raw", g_raw), ("omega_r_raw", omega_r_raw)):
        if value.dtype not in (torch.bfloat16, torch.float32):
            raise TypeError(f"{name} must be bf16 or fp32, got {value.dtype}")
    if any(value.dtype != torch.float32 for value in inputs[2:]):
        raise TypeError("omega_bias, r_bias, A_log, dt_bias, and initial_precision_param must be FP32")
    for name, value in (("omega_min", omega_min), ("r_min", r_min)):
        if not isinstance(value, (int, float)):
            raise TypeError(f"{name} must be a Python scalar, got {type(value).__name__}")
        if not math.isfinite(float(value)):
            raise ValueError(f"{name} must be finite, got {value!r}")
    if K > 256:
        raise ValueError(f"the iso gate supports K <= 256, got {K}")
    return B, T, H, K


def _iso_kdn_gate_precumsum_fwd(g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias,
                                initial_precision_param, omega_min, r_min):
    B, T, H, K = g_raw.shape
    dev = g_raw.device
    g_cumsum = torch.empty((B, T, H, K), device=dev, dtype=torch.float32)
    a = torch.empty((B, T, H), device=dev, dtype=torch.float32)
    omega = torch.empty_like(a)
    r = torch.empty_like(a)
    mu = torch.empty((H,), device=dev, dtype=torch.float32)
    with torch.cuda.device(dev):
        _lib.call("kdn_iso_gate_fwd", _lib.ptr(g_raw), _lib.is_bf16(g_raw), _lib.ptr(omega_r_raw),
                  _lib.is_bf16(omega_r_raw), omega_r_raw.stride(0), omega_r_raw.stride(1),
                  _lib.ptr(omega_bias), _lib.ptr(r_bias), _lib.ptr(A_log), _lib.ptr(dt_bias),
                  _lib.ptr(initial_precision_param), float(omega_min), float(r_min), B, T, H, K,
                  ISO_GATE_CHUNK_SIZE, _lib.ptr(g_cumsum), _lib.ptr(a), _lib.ptr(omega), _lib.ptr(r),
                  _lib.ptr(mu), _lib.stream_of(g_raw))
    return g_cumsum, a, omega, r, mu


def _iso_kdn_gate_precumsum_bwd(g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias,
                                initial_precision_param, a, dg_pre_reverse, da, domega, dr,
                                d_initial_precision, needs_input_grad):
    """Reference iso_kdn_chunk.py:1116-1314."""
    B, T, H, K = g_raw.shape
    (need_dg_raw, need_domega_r_raw, need_domega_bias, need_dr_bias, need_dA_log, need_ddt_bias,
     need_dmu) = needs_input_grad
    dev = g_raw.device
    if B == 0 or T == 0:
        dmu = None
        if need_dmu:
            dmu = (torch.zeros_like(initial_precision_param) if d_initial_precision is None
                   else d_initial_precision.float() * torch.sigmoid(initial_precision_param))
        return (torch.zeros_like(g_raw) if need_dg_raw else None,
                torch.zeros_like(omega_r_raw) if need_domega_r_raw else None,
                torch.zeros_like(omega_bias) if need_domega_bias else None,
                torch.zeros_like(r_bias) if need_dr_bias else None,
                torch.zeros_like(A_log) if need_dA_log else None,
                torch.zeros_like(dt_bias) if need_ddt_bias else None, dmu)
    if dg_pre_reverse is not None:
        if dg_pre_reverse.shape != g_raw.shape:
            raise ValueError(f"dg_pre_reverse must have shape {tuple(g_raw.shape)}, "
                             f"got {tuple(dg_pre_reverse.shape)}")
        dg_pre_reverse = dg_pre_reverse.float().contiguous()
    for name, value in (("da", da), ("domega", domega), ("dr", dr)):
        if value is not None and value.shape != (B, T, H):
            raise ValueError(f"{name} must have shape {(B, T, H)}, got {tuple(value.shape)}")
    da = da.float().contiguous() if da is not None else None
    domega = domega.float().contiguous() if domega is not None else None
    dr = dr.float().contiguous() if dr is not None else None
    if d_initial_precision is not None:
        if d_initial_precision.shape != (H,):
            raise ValueError(f"d_initial_precision must have shape {(H,)}, "
                             f"got {tuple(d_initial_precision.shape)}")
        d_initial_precision = d_initial_precision.float().contiguous()
    dg_raw = torch.empty_like(g_raw) if need_dg_raw else None
    domega_r_raw = (torch.empty(omega_r_raw.shape, device=dev, dtype=omega_r_raw.dtype)
                    if need_domega_r_raw else None)
    domega_bias = torch.empty((H,), device=dev, dtype=torch.float32) if need_domega_bias else None
    dr_bias = torch.empty((H,), device=dev, dtype=torch.float32) if need_dr_bias else None
    dA_log = torch.empty((H,), device=dev, dtype=torch.float32) if need_dA_log else None
    ddt_bias = torch.empty((H * K,), device=dev, dtype=torch.float32) if need_ddt_bias else None
    dmu = torch.empty((H,), device=dev, dtype=torch.float32) if need_dmu else None
    ws_bytes = _lib.size("kdn_iso_gate_bwd_workspace_size", B, T, H, K, ISO_GATE_CHUNK_SIZE)
    ws = torch.empty((ws_bytes,), device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        _lib.call("kdn_iso_gate_bwd", _lib.ptr(g_raw), _lib.is_bf16(g_raw), _lib.ptr(omega_r_raw),
                  _lib.is_bf16(omega_r_raw), omega_r_raw.stride(0), omega_r_raw.stride(1),
                  _lib.ptr(omega_bias), _lib.ptr(r_bias), _lib.ptr(A_log), _lib.ptr(dt_bias),
                  _lib.ptr(initial_precision_param), _lib.ptr(dg_pre_reverse), _lib.ptr(da),
                  _lib.ptr(domega), _lib.ptr(dr), _lib.ptr(d_initial_precision), B, T, H, K,
                  ISO_GATE_CHUNK_SIZE, _lib.ptr(dg_raw), _lib.ptr(domega_r_raw), _lib.ptr(dA_log),
                  _lib.ptr(ddt_bias), _lib.ptr(domega_bias), _lib.ptr(dr_bias), _lib.ptr(dmu),
                  _lib.ptr(ws), ws_bytes, _lib.stream_of(g_raw))
    return dg_raw, domega_r_raw, domega_bias, dr_bias, dA_log, ddt_bias, dmu


class _IsoKDNGatePrecumsumFunction(torch.autograd.Function):
    """Reference iso_kdn_chunk.py:1317-1392."""

    @staticmethod
    def forward(ctx, g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias, initial_precision_param,
                omega_min, r_min):
        g_cumsum, a, omega, r, mu = _iso_kdn_gate_precumsum_fwd(
            g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias, initial_precision_param, omega_min, r_min)
        ctx.save_for_backward(g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias, initial_precision_param, a)
        ctx.set_materialize_grads(False)
        return g_cumsum, a, omega, r, mu

    @staticmethod
    def backward(ctx, dg_pre_reverse, da, domega, dr, d_initial_precision):
        g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias, mu_param, a = ctx.saved_tensors
        grads = _iso_kdn_gate_precumsum_bwd(g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias, mu_param,
                                            a, dg_pre_reverse, da, domega, dr, d_initial_precision,
                                            ctx.needs_input_grad[:7])
        return (*grads, None, None)


@torch.compiler.disable
def _iso_kdn_gate_precumsum_paired(g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias,
                                   initial_precision_param, omega_min, r_min):
    """Return private paired ``(base2_prefix, a, omega, r, initial_precision)`` tensors.

    ``base2_prefix`` is the chunk-local (64 tokens) inclusive prefix of the per-channel
    log-gate in base 2 and must have exactly one consumer, ``_chunk_kda_precumsum_paired``:
    that Function returns a natural-log-coordinate cotangent which this Function's backward
    reverse-sums within the chunk (reference iso_kdn_chunk.py:1395-1436, 927-936).
    """
    _validate_iso_gate_inputs(g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias,
                              initial_precision_param, omega_min, r_min)
    return _IsoKDNGatePrecumsumFunction.apply(
        g_raw.contiguous(), omega_r_raw, omega_bias.contiguous(), r_bias.contiguous(), A_log.contiguous(),
        dt_bias.contiguous(), initial_precision_param.contiguous(), float(omega_min), float(r_min))


# ---------------------------------------------------------------------------
# Scalar Kalman gain
# ---------------------------------------------------------------------------

def _require_same_cuda_device(a, *named_tensors):
    """Reference iso_kdn_chunk.py:1446-1461."""
    if not a.is_cuda:
        raise ValueError(f"a must be a GPU tensor; got device={a.device}")
    device = a.device
    for name, tensor in named_tensors:
        if not tensor.is_cuda:
            raise ValueError(f"{name} must be a GPU tensor; got device={tensor.device}")
        if tensor.device != device:
            raise ValueError(f"all tensors must share a GPU device; a is on {device}, "
                             f"but {name} is on {tensor.device}")
    return device


def _posterior_scale(head_dim, info_scale):
    """s = info_scale / head_dim with the reference's checks (iso_kdn_chunk.py:2002-2020)."""
    if isinstance(head_dim, bool) or not isinstance(head_dim, int):
        raise TypeError(f"head_dim must be a positive int, got {type(head_dim).__name__}")
    if head_dim <= 0:
        raise ValueError(f"head_dim must be positive, got {head_dim}")
    if info_scale is None:
        resolved = float(head_dim)
    else:
        if isinstance(info_scale, bool) or not isinstance(info_scale, Real):
            raise TypeError(f"info_scale must be a positive finite real, got {type(info_scale).__name__}")
        resolved = float(info_scale)
        if not math.isfinite(resolved) or resolved <= 0:
            raise ValueError(f"info_scale must be positive and finite, got {info_scale!r}")
    return resolved / float(head_dim)


def _iso_kdn_gain_forward(a, omega, r, initial_precision, *, out_dtype, save_state, posterior_scale,
                          output_final_state=False):
    """Returns (beta, p_prev or None, final_precision [B,H] or None).  ``initial_precision`` is
    [H] (the reference's form) or [B,H] (continuation of an earlier segment)."""
    B, T, H = a.shape
    device = _require_same_cuda_device(a, ("omega", omega), ("r", r), ("initial_precision", initial_precision))
    prec_mode = 0 if initial_precision.ndim == 1 else 1
    gain = torch.empty((B, T, H), dtype=torch.float32, device=device)
    p_prev = torch.empty((B, T, H), dtype=torch.float32, device=device) if save_state else None
    fprec = None
    if output_final_state:
        fprec = torch.empty((B, H), dtype=torch.float32, device=device)
        if T == 0:
            fprec.copy_(initial_precision.float().expand(B, H))
    if T > 0 and B > 0:
        ws_bytes = _lib.size("kdn_iso_gain_workspace_size", B, T, H)
        ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=device)
        with torch.cuda.device(device):
            _lib.call("kdn_iso_gain_fwd", _lib.ptr(a), _lib.ptr(omega), _lib.ptr(r),
                      _lib.ptr(initial_precision), prec_mode, B, T, H, float(posterior_scale), _lib.ptr(gain),
                      _lib.ptr(p_prev), _lib.ptr(fprec), _lib.ptr(ws), ws_bytes, _lib.stream_of(a))
    return (gain if out_dtype == torch.float32 else gain.to(out_dtype)), p_prev, fprec


def _iso_kdn_gain_backward(a, omega, r, initial_precision, dgain, p_prev, *, posterior_scale,
                           final_precision=None, d_final_precision=None):
    B, T, H = a.shape
    device = _require_same_cuda_device(a, ("omega", omega), ("r", r), ("initial_precision", initial_precision),
                                       ("dgain", dgain), ("previous_covariance", p_prev))
    prec_mode = 0 if initial_precision.ndim == 1 else 1
    da = torch.empty_like(a)
    domega = torch.empty_like(omega)
    dr = torch.empty_like(r)
    # the backward carry kernel writes every entry of dmu; only the token-free case needs zeros
    dmu = (torch.empty if (T > 0 and B > 0) else torch.zeros)(initial_precision.shape, dtype=torch.float32,
                                                              device=device)
    if T > 0 and B > 0:
        ws_bytes = _lib.size("kdn_iso_gain_workspace_size", B, T, H)
        ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=device)
        dfp = d_final_precision.float().contiguous() if d_final_precision is not None else None
        with torch.cuda.device(device):
            _lib.call("kdn_iso_gain_bwd", _lib.ptr(a), _lib.ptr(omega), _lib.ptr(r), _lib.ptr(initial_precision),
                      prec_mode, _lib.ptr(dgain), _lib.ptr(p_prev), _lib.ptr(final_precision if dfp is not None
                                                                             else None),
                      _lib.ptr(dfp), B, T, H, float(posterior_scale), _lib.ptr(da), _lib.ptr(domega), _lib.ptr(dr),
                      _lib.ptr(dmu), _lib.ptr(ws), ws_bytes, _lib.stream_of(a))
    elif d_final_precision is not None and B > 0:
        # no tokens: the final precision is the initial one
        dfp = d_final_precision.float()
        dmu.copy_(dfp if prec_mode else dfp.sum(0))
    return da, domega, dr, dmu.to(initial_precision.dtype)


class _IsoKDNGainFunction(torch.autograd.Function):
    """Reference iso_kdn_chunk.py:1896-1962, plus the optional final precision output."""

    @staticmethod
    def forward(ctx, a, omega, r, initial_precision, out_dtype, posterior_scale, needs_backward,
                output_final_state=False):
        gain, p_prev, fprec = _iso_kdn_gain_forward(a, omega, r, initial_precision, out_dtype=out_dtype,
                                                    save_state=needs_backward, posterior_scale=posterior_scale,
                                                    output_final_state=output_final_state)
        ctx.posterior_scale = posterior_scale
        ctx.has_saved_state = needs_backward
        if needs_backward:
            ctx.save_for_backward(a, omega, r, initial_precision, p_prev, fprec)
        if output_final_state:
            return gain, fprec
        return gain

    @staticmethod
    def backward(ctx, dgain, d_final_precision=None):
        if dgain is None and d_final_precision is None:
            return None, None, None, None, None, None, None, None
        if not ctx.has_saved_state:
            raise RuntimeError("Isotropic KDN gain backward called after a no-save forward")
        a, omega, r, initial_precision, p_prev, fprec = ctx.saved_tensors
        dgain = torch.zeros_like(a) if dgain is None else dgain.float().contiguous()
        da, domega, dr, dmu = _iso_kdn_gain_backward(a, omega, r, initial_precision, dgain, p_prev,
                                                     posterior_scale=ctx.posterior_scale, final_precision=fprec,
                                                     d_final_precision=d_final_precision)
        needs = ctx.needs_input_grad
        return (da if needs[0] else None, domega if needs[1] else None, dr if needs[2] else None,
                dmu if needs[3] else None, None, None, None, None)


@torch.compiler.disable
def iso_kdn_gain(a, omega, r, initial_precision, *, head_dim, out_dtype=None, info_scale=None,
                 output_final_state=False):
    """Differentiable Isotropic KDN scalar write gate beta [B,T,H] (reference :1965-2031).

    z = a p + omega;  beta = z / (r + z);  p' = r z / (r + s z),  s = info_scale / head_dim,
    p_0 = 1 / initial_precision.  Keys are unit-normalised on the production path, so |k|^2 = 1.

    State continuation (not in the reference, which takes only [H]): ``initial_precision`` may be
    [B,H], and ``output_final_state=True`` returns ``(beta, final_precision [B,H] fp32)`` with
    final_precision = 1 / p_T, so a sequence split into segments gives the beta of the whole when
    each segment starts from the previous segment's final precision.  Gradients flow through both.
    """
    if a.ndim != 3:
        raise ValueError(f"a must have shape [B,T,H], got {tuple(a.shape)}")
    if omega.shape != a.shape or r.shape != a.shape:
        raise ValueError("a, omega, and r must share shape [B,T,H]; got "
                         f"a={tuple(a.shape)}, omega={tuple(omega.shape)}, r={tuple(r.shape)}")
    B, _, H = a.shape
    if initial_precision.shape not in ((H,), (B, H)):
        raise ValueError(f"initial_precision must have shape [{H}] or [{B},{H}], "
                         f"got {tuple(initial_precision.shape)}")
    _require_same_cuda_device(a, ("omega", omega), ("r", r), ("initial_precision", initial_precision))
    if out_dtype is None:
        out_dtype = torch.float32
    posterior_scale = _posterior_scale(head_dim, info_scale)
    needs_backward = torch.is_grad_enabled() and any(
        t.requires_grad for t in (a, omega, r, initial_precision))
    return _IsoKDNGainFunction.apply(a.float().contiguous(), omega.float().contiguous(), r.float().contiguous(),
                                     initial_precision.float().contiguous(), out_dtype, posterior_scale,
                                     needs_backward, bool(output_final_state))


# ---------------------------------------------------------------------------
# Fused front: gate frontend -> scalar gain
# ---------------------------------------------------------------------------

class _IsoKDNFrontFunction(torch.autograd.Function):
    """``_iso_kdn_gate_precumsum_paired`` -> ``iso_kdn_gain`` (reference iso_kdn_chunk.py:1317-1392,
    1896-1962, composed as lit_gpt/iso_kdn.py:277-304) as one op.  Forward: the gate's kernel also
    writes each 64-token chunk's gain map, and one gain kernel carries them; backward: the gain's
    reverse chunk maps, then the gate's backward kernel runs the gain's per-chunk backward itself, so
    the cotangents of a, omega, r never reach memory.  Returns (g_cumsum, beta[, final_precision])."""

    @staticmethod
    def forward(ctx, g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias, mu_param, initial_precision,
                omega_min, r_min, posterior_scale, needs_backward, output_final_state):
        B, T, H, K = g_raw.shape
        dev = g_raw.device
        g_cumsum = torch.empty((B, T, H, K), device=dev, dtype=torch.float32)
        a = torch.empty((B, T, H), device=dev, dtype=torch.float32)
        omega = torch.empty_like(a)
        r = torch.empty_like(a)
        beta = torch.empty_like(a)
        mu = torch.empty((H,), device=dev, dtype=torch.float32)
        p_prev = torch.empty_like(a) if needs_backward else None
        fprec = torch.empty((B, H), device=dev, dtype=torch.float32) if output_final_state else None
        prec_mode = 0 if initial_precision is None or initial_precision.ndim == 1 else 1
        ws_bytes = _lib.size("kdn_iso_front_workspace_size", B, T, H, K)
        ws = torch.empty((ws_bytes,), device=dev, dtype=torch.uint8)
        with torch.cuda.device(dev):
            _lib.call("kdn_iso_front_fwd", _lib.ptr(g_raw), _lib.is_bf16(g_raw), _lib.ptr(omega_r_raw),
                      _lib.is_bf16(omega_r_raw), omega_r_raw.stride(0), omega_r_raw.stride(1),
                      _lib.ptr(omega_bias), _lib.ptr(r_bias), _lib.ptr(A_log), _lib.ptr(dt_bias),
                      _lib.ptr(mu_param), float(omega_min), float(r_min), _lib.ptr(initial_precision), prec_mode,
                      B, T, H, K, float(posterior_scale), _lib.ptr(g_cumsum), _lib.ptr(a), _lib.ptr(omega),
                      _lib.ptr(r), _lib.ptr(mu), _lib.ptr(beta), _lib.ptr(p_prev), _lib.ptr(fprec), _lib.ptr(ws),
                      ws_bytes, _lib.stream_of(g_raw))
        ctx.posterior_scale = posterior_scale
        ctx.has_saved_state = needs_backward
        if needs_backward:
            ctx.save_for_backward(g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias, mu_param,
                                  initial_precision, a, omega, r, mu, p_prev, fprec)
        ctx.set_materialize_grads(False)
        return (g_cumsum, beta, fprec) if output_final_state else (g_cumsum, beta)

    @staticmethod
    def backward(ctx, d_g_cumsum, d_beta, d_final_precision=None):
        if not ctx.has_saved_state:
            raise RuntimeError("Isotropic KDN front backward called after a no-save forward")
        (g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias, mu_param, initial_precision, a, omega, r, mu,
         p_prev, fprec) = ctx.saved_tensors
        B, T, H, K = g_raw.shape
        dev = g_raw.device
        needs = ctx.needs_input_grad
        prec_mode = 0 if initial_precision is None or initial_precision.ndim == 1 else 1
        dg_pre = d_g_cumsum.float().contiguous() if d_g_cumsum is not None else None
        dbeta = torch.zeros_like(a) if d_beta is None else d_beta.float().contiguous()
        dfp = d_final_precision.float().contiguous() if d_final_precision is not None else None
        dg_raw = torch.empty_like(g_raw) if needs[0] else None
        domega_r_raw = (torch.empty(omega_r_raw.shape, device=dev, dtype=omega_r_raw.dtype)
                        if needs[1] else None)
        domega_bias = torch.empty((H,), device=dev, dtype=torch.float32) if needs[2] else None
        dr_bias = torch.empty((H,), device=dev, dtype=torch.float32) if needs[3] else None
        dA_log = torch.empty((H,), device=dev, dtype=torch.float32) if needs[4] else None
        ddt_bias = torch.empty((H * K,), device=dev, dtype=torch.float32) if needs[5] else None
        dmu = torch.empty((H,), device=dev, dtype=torch.float32) if needs[6] else None
        dinit = (torch.empty_like(initial_precision) if initial_precision is not None and needs[7] else None)
        ws_bytes = _lib.size("kdn_iso_front_workspace_size", B, T, H, K)
        ws = torch.empty((ws_bytes,), device=dev, dtype=torch.uint8)
        with torch.cuda.device(dev):
            _lib.call("kdn_iso_front_bwd", _lib.ptr(g_raw), _lib.is_bf16(g_raw), _lib.ptr(omega_r_raw),
                      _lib.is_bf16(omega_r_raw), omega_r_raw.stride(0), omega_r_raw.stride(1),
                      _lib.ptr(omega_bias), _lib.ptr(r_bias), _lib.ptr(A_log), _lib.ptr(dt_bias),
                      _lib.ptr(mu_param), _lib.ptr(initial_precision), prec_mode, _lib.ptr(a), _lib.ptr(omega),
                      _lib.ptr(r), _lib.ptr(mu), _lib.ptr(p_prev), _lib.ptr(fprec if dfp is not None else None),
                      _lib.ptr(dg_pre), _lib.ptr(dbeta), _lib.ptr(dfp), B, T, H, K, float(ctx.posterior_scale),
                      _lib.ptr(dg_raw), _lib.ptr(domega_r_raw), _lib.ptr(dA_log), _lib.ptr(ddt_bias),
                      _lib.ptr(domega_bias), _lib.ptr(dr_bias), _lib.ptr(dmu), _lib.ptr(dinit), _lib.ptr(ws),
                      ws_bytes, _lib.stream_of(g_raw))
        return (dg_raw, domega_r_raw, domega_bias, dr_bias, dA_log, ddt_bias, dmu, dinit,
                None, None, None, None, None)


@torch.compiler.disable
def iso_kdn_front(g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias, initial_precision_param, omega_min,
                  r_min, *, head_dim, info_scale=None, initial_precision=None, output_final_state=False):
    """``_iso_kdn_gate_precumsum_paired`` -> ``iso_kdn_gain`` as the iso layer composes them (reference
    lit_gpt/iso_kdn.py:277-304), fused: returns ``(g_cumsum, beta)`` (plus ``final_precision`` [B,H]
    with ``output_final_state``), equal to the two ops' outputs with ``out_dtype=torch.float32``.  The
    gain's prior precision is the gate's ``0.1 + softplus(initial_precision_param)`` unless
    ``initial_precision`` ([H] or [B,H], state continuation) is given.  ``g_cumsum`` keeps the gate's
    contract: its one consumer is ``_chunk_kda_precumsum_paired``.  Same argument checks and errors as
    the two ops."""
    B, T, H, K = _validate_iso_gate_inputs(g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias,
                                           initial_precision_param, omega_min, r_min)
    if initial_precision is not None:
        if not isinstance(initial_precision, torch.Tensor):
            raise TypeError("initial_precision must be a torch.Tensor")
        if initial_precision.shape not in ((H,), (B, H)):
            raise ValueError(f"initial_precision must have shape [{H}] or [{B},{H}], "
                             f"got {tuple(initial_precision.shape)}")
        _require_same_cuda_device(g_raw, ("initial_precision", initial_precision))
    posterior_scale = _posterior_scale(head_dim, info_scale)
    if B == 0 or T == 0:  # nothing to fuse: the two ops
        g_cumsum, a, omega, r, mu = _iso_kdn_gate_precumsum_paired(
            g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias, initial_precision_param, omega_min, r_min)
        out = iso_kdn_gain(a, omega, r, mu if initial_precision is None else initial_precision, head_dim=head_dim,
                           out_dtype=torch.float32, info_scale=info_scale, output_final_state=output_final_state)
        return (g_cumsum, *out) if output_final_state else (g_cumsum, out)
    init = initial_precision.float().contiguous() if initial_precision is not None else None
    needs_backward = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad
        for t in (g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias, initial_precision_param, init))
    return _IsoKDNFrontFunction.apply(
        g_raw.contiguous(), omega_r_raw, omega_bias.contiguous(), r_bias.contiguous(), A_log.contiguous(),
        dt_bias.contiguous(), initial_precision_param.contiguous(), init, float(omega_min), float(r_min),
        posterior_scale, needs_backward, bool(output_final_state))


# ---------------------------------------------------------------------------
# Chunked memory scan (KDA form, kappa = beta k)
# ---------------------------------------------------------------------------

def _l2norm_fwd(x):
    rows = x.numel() // x.shape[-1]
    y = torch.empty(x.shape, device=x.device, dtype=torch.bfloat16)
    rstd = torch.empty(x.shape[:-1], device=x.device, dtype=torch.float32)
    _lib.call("kdn_l2norm_fwd", _lib.ptr(x), _lib.is_bf16(x), rows, x.shape[-1], _L2NORM_EPS, _lib.ptr(y), 1,
              _lib.ptr(rstd), _lib.stream_of(x))
    return y, rstd


def _l2norm_bwd(x, rstd, dy):
    rows = x.numel() // x.shape[-1]
    dx = torch.empty_like(x)
    _lib.call("kdn_l2norm_bwd", _lib.ptr(x), _lib.is_bf16(x), _lib.ptr(rstd), _lib.ptr(dy), _lib.is_bf16(dy),
              rows, x.shape[-1], _lib.ptr(dx), _lib.stream_of(x))
    return dx


def _chunk_kda_fwd_precum(q, k, v, g_cumsum, beta, scale, *, initial_state=None, output_final_state=False,
                          out_dtype=torch.bfloat16, need_backward=True, q_rstd=None, k_rstd=None):
    """Memory scan forward on normalised bf16 q, k (reference :2037-2086); kappa = beta k.  With
    need_backward=False the returned saved buffer cannot feed _chunk_kda_bwd_precum.  With q_rstd /
    k_rstd (f32 [B,T,H], filled here) q, k are raw and the scan applies the in-op L2 norm itself."""
    return _memscan.mem_fwd(q, k, beta, True, v, g_cumsum, scale, initial_state=initial_state,
                            output_final_state=output_final_state, out_dtype=out_dtype,
                            need_backward=need_backward, q_rstd=q_rstd, k_rstd=k_rstd)


def _chunk_kda_bwd_precum(q, k, v, g_cumsum, beta, saved, scale, do, *, d_final_state=None,
                          need_initial_state_grad=False, q_rstd=None, k_rstd=None):
    """Memory scan backward (reference :2089-2187): natural-log dg, no reverse cumsum.  With q_rstd /
    k_rstd (the in-op L2 norm's, from the forward; q and k the raw inputs) dq, dk are returned for the
    raw inputs, the norm's backward included."""
    return _memscan.mem_bwd(q, k, beta, True, v, g_cumsum, saved, scale, do, d_final_state=d_final_state,
                            need_initial_state_grad=need_initial_state_grad, q_rstd=q_rstd, k_rstd=k_rstd)


class _ChunkKDAPrecumsumFunction(torch.autograd.Function):
    """Reference iso_kdn_chunk.py:2190-2238: L2-normalise q, k inside; memory scan; VJPs.  With an
    initial state h0 [B,H,K,V] and / or the final state requested, their gradients flow too.

    For bf16 q, k the norm runs inside the scan: the forward normalises the rows of the raw q, k as
    it loads them and writes their rstd, and the backward forms the normalised operands again and
    applies the norm's backward in its kernel.  fp32 q, k keep kdn_l2norm_fwd / kdn_l2norm_bwd.

    In the "recompute" backward mode (_memscan.set_backward_mode) the forward keeps only its inputs
    and the rows' rstd, and the backward rebuilds the scan's intermediates first (same gradients)."""

    @staticmethod
    def forward(ctx, q, k, v, g_cumsum, beta, scale, initial_state=None, output_final_state=False):
        dev = q.device
        ctx.fused_norm = q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16
        need_backward = any(ctx.needs_input_grad)
        ctx.recompute = need_backward and _memscan.backward_mode() == "recompute"
        keep = need_backward and not ctx.recompute  # the forward's intermediates feed the backward
        with torch.cuda.device(dev):
            vb = v if v.dtype == torch.bfloat16 else v.to(torch.bfloat16)
            out_dtype = q.dtype if q.dtype == torch.float32 else torch.bfloat16
            if ctx.fused_norm:
                q = q.contiguous()
                k = k.contiguous()
                q_rstd = torch.empty(q.shape[:-1], device=dev, dtype=torch.float32)
                k_rstd = torch.empty(k.shape[:-1], device=dev, dtype=torch.float32)
                o, saved, ht = _chunk_kda_fwd_precum(q, k, vb.contiguous(), g_cumsum, beta, scale,
                                                     initial_state=initial_state,
                                                     output_final_state=output_final_state, out_dtype=out_dtype,
                                                     need_backward=keep, q_rstd=q_rstd, k_rstd=k_rstd)
            else:
                qn, q_rstd = _l2norm_fwd(q)
                kn, k_rstd = _l2norm_fwd(k)
                o, saved, ht = _chunk_kda_fwd_precum(qn, kn, vb.contiguous(), g_cumsum, beta, scale,
                                                     initial_state=initial_state,
                                                     output_final_state=output_final_state, out_dtype=out_dtype,
                                                     need_backward=keep)
        saved = saved if keep else None
        h0 = initial_state if ctx.recompute else None  # the state pass starts from it again
        if ctx.fused_norm:
            ctx.save_for_backward(q, q_rstd, k, k_rstd, vb, g_cumsum, beta, saved, h0)
        else:
            ctx.save_for_backward(q, q_rstd, qn, k, k_rstd, kn, vb, g_cumsum, beta, saved, h0)
        ctx.scale = scale
        ctx.h0_dtype = initial_state.dtype if initial_state is not None else None
        o = o if o.dtype == q.dtype else o.to(q.dtype)
        return (o, ht) if output_final_state else o

    @staticmethod
    def backward(ctx, do, dht=None):
        need_h0 = ctx.h0_dtype is not None and ctx.needs_input_grad[6]
        with torch.cuda.device(do.device):
            if ctx.fused_norm:
                q, q_rstd, k, k_rstd, vb, g_cumsum, beta, saved, h0 = ctx.saved_tensors
                if ctx.recompute:
                    saved = _memscan.rebuild_saved(q, k, beta, True, vb, g_cumsum, ctx.scale, initial_state=h0,
                                                   fused_norm=True)
                dq, dk, dv, db, dg, dh0 = _chunk_kda_bwd_precum(q, k, vb, g_cumsum, beta, saved, ctx.scale, do,
                                                                d_final_state=dht, need_initial_state_grad=need_h0,
                                                                q_rstd=q_rstd, k_rstd=k_rstd)
            else:
                q, q_rstd, qn, k, k_rstd, kn, vb, g_cumsum, beta, saved, h0 = ctx.saved_tensors
                if ctx.recompute:
                    saved = _memscan.rebuild_saved(qn, kn, beta, True, vb, g_cumsum, ctx.scale, initial_state=h0)
                dqn, dkn, dv, db, dg, dh0 = _chunk_kda_bwd_precum(qn, kn, vb, g_cumsum, beta, saved, ctx.scale, do,
                                                                  d_final_state=dht, need_initial_state_grad=need_h0)
                dq = _l2norm_bwd(q, q_rstd, dqn)
                dk = _l2norm_bwd(k, k_rstd, dkn)
        dh0 = dh0.to(ctx.h0_dtype) if dh0 is not None else None
        return dq, dk, dv, dg, db, None, dh0, None


@torch.compiler.disable
def _chunk_kda_precumsum_paired(q, k, v, g_cumsum, beta, scale=None, *, initial_state=None,
                                output_final_state=False):
    """Consume the private paired cumulative gate on the fixed-length path (reference :2241-2285).

    ``g_cumsum`` must be the unbranched output of :func:`_iso_kdn_gate_precumsum_paired`.
    Returns o [B,T,H,V] in q's dtype; the backward returns the natural-log-coordinate gate
    cotangent expected by that producer.

    State continuation (the reference's wrapper passes no state): ``initial_state`` [B,H,K,V]
    starts the memory from an earlier segment's state, and ``output_final_state=True`` returns
    ``(o, final_state [B,H,K,V] fp32)``.
    """
    if q.ndim != 4 or q.shape != k.shape:
        raise ValueError(f"q and k must share [B,T,H,K], got {tuple(q.shape)} and {tuple(k.shape)}")
    B, T, H, K = q.shape
    if min(B, T, H, K) == 0:
        raise ValueError("_chunk_kda_precumsum_paired requires non-empty B,T,H,K dimensions")
    if v.ndim != 4 or v.shape[:3] != (B, T, H):
        raise NotImplementedError("_chunk_kda_precumsum_paired does not support GVA; v must have q's B,T,H")
    if v.shape[-1] == 0:
        raise ValueError("_chunk_kda_precumsum_paired requires a non-empty value dimension")
    if g_cumsum.shape != (B, T, H, K):
        raise ValueError(f"g_cumsum must have shape {(B, T, H, K)}, got {tuple(g_cumsum.shape)}")
    if beta.shape != (B, T, H):
        raise ValueError(f"beta must have shape {(B, T, H)}, got {tuple(beta.shape)}")
    if K > 256:
        raise ValueError(f"KDA supports key head dimension <=256, got {K}")
    if K not in (64, 128) or v.shape[-1] not in (64, 128):
        raise ValueError(f"the MI355X scan supports K, V in {{64, 128}}, got K={K}, V={v.shape[-1]}")
    if g_cumsum.dtype != torch.float32:
        raise TypeError(f"g_cumsum must be FP32 base-2 cumulative gate, got {g_cumsum.dtype}")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"q, k, and v must share a dtype, got {q.dtype}, {k.dtype}, {v.dtype}")
    if q.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"q, k, v must be bf16 or fp32, got {q.dtype}")
    tensors = (q, k, v, g_cumsum, beta)
    if not all(x.is_cuda for x in tensors):
        raise ValueError("_chunk_kda_precumsum_paired is GPU-only")
    if len({x.device for x in tensors}) != 1:
        raise ValueError("all _chunk_kda_precumsum_paired tensors must be on the same GPU device")
    if initial_state is not None:
        if initial_state.shape != (B, H, K, v.shape[-1]) or initial_state.device != q.device:
            raise ValueError(f"initial_state must be a tensor of shape {(B, H, K, v.shape[-1])} on {q.device}")
        if initial_state.dtype != torch.float32:
            raise TypeError(f"initial_state must be fp32, got {initial_state.dtype}")
    if scale is None:
        scale = K ** -0.5
    return _ChunkKDAPrecumsumFunction.apply(q.contiguous(), k.contiguous(), v.contiguous(),
                                            g_cumsum.contiguous(), beta.float().contiguous(), scale,
                                            initial_state.contiguous() if initial_state is not None else None,
                                            bool(output_final_state))


__all__ = ("_chunk_kda_precumsum_paired", "_iso_kdn_gate_precumsum_paired", "iso_kdn_gain", "qkv_causal_conv1d")
