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

import math

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


def kdn_kalman_step(q, k, v, g_cumsum, *, state, precision, omega, r, info_scale, a=None, alpha=None, k_gain=None,
                    scale=None, out_dtype=None, precision_out=None):
    """One token of the whole Kalman step (gain from the carried precision + memory update) in one
    launch (``kdn_kalman_step``).  Advances ``state`` [B,H,K,V] fp32 in place and returns
    ``(o [B,1,H,V], new_precision)``; ``new_precision`` is written to ``precision_out`` when given
    (it must not be ``precision``).

    Isotropic form: ``a`` (mean alpha^2), ``omega``, ``r`` [B,1,H]; ``precision`` [B,H]; q, k are
    L2-normalised inside and the production gain's unit-key form is used (as
    :func:`iso_kdn_gain` does): z = a/c + omega, beta = z/(r+z), c' = (r + s z)/(r z),
    s = info_scale / K.  Diagonal form: ``alpha`` (unclamped, the gain's input), ``omega``
    [B,1,H,K], ``r`` [B,1,H], ``k_gain`` [B,1,H,K] fp32 (defaults to k), ``precision`` [B,H,K];
    q, k already normalised.  ``g_cumsum`` [B,1,H,K] fp32 is the memory's base-2 log decay.
    """
    if (a is None) == (alpha is None):
        raise ValueError("pass exactly one of a (isotropic) or alpha (diagonal)")
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
    iso = a is not None
    gain_a = a if iso else alpha
    tok = (B, 1, H) if iso else (B, 1, H, K)
    prec_shape = (B, H) if iso else (B, H, K)
    for name, x, shp in (("a" if iso else "alpha", gain_a, tok), ("omega", omega, tok), ("r", r, (B, 1, H)),
                         ("precision", precision, prec_shape)):
        if tuple(x.shape) != shp:
            raise ValueError(f"{name} must have shape {shp}, got {tuple(x.shape)}")
    if not iso and k_gain is not None and tuple(k_gain.shape) != (B, 1, H, K):
        raise ValueError(f"k_gain must have shape {(B, 1, H, K)}, got {tuple(k_gain.shape)}")
    if not (float(info_scale) > 0 and math.isfinite(float(info_scale))):
        raise ValueError(f"info_scale must be positive and finite, got {info_scale!r}")
    if q.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"q must be bf16 or fp32, got {q.dtype}")
    out_dtype = q.dtype if out_dtype is None else out_dtype
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"out_dtype must be bf16 or fp32, got {out_dtype}")
    _lib.require_device(q, k, v, g_cumsum, state, precision, gain_a, omega, r, k_gain, precision_out)
    dt = q.dtype
    q, k, v = (x.to(dt).contiguous() for x in (q, k, v))
    gain_a, omega, r, pin = (x.float().contiguous() for x in (gain_a, omega, r, precision))
    kg = k_gain.float().contiguous() if (k_gain is not None and not iso) else None
    if precision_out is None:
        precision_out = torch.empty(prec_shape, device=q.device, dtype=torch.float32)
    elif (precision_out.shape != prec_shape or precision_out.dtype != torch.float32
          or not precision_out.is_contiguous() or precision_out.data_ptr() == pin.data_ptr()):
        raise ValueError("precision_out must be a contiguous fp32 tensor of the precision's shape, distinct from it")
    o = torch.empty((B, 1, H, V), device=q.device, dtype=out_dtype)
    scale = K ** -0.5 if scale is None else float(scale)
    with torch.cuda.device(q.device):
        _lib.call("kdn_kalman_step", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.is_bf16(q), _lib.ptr(g_cumsum.contiguous()),
                  _lib.ptr(gain_a), _lib.ptr(omega), _lib.ptr(r), _lib.ptr(kg), _lib.ptr(pin), _lib.ptr(precision_out),
                  int(iso), B, H, K, V, scale, float(info_scale), _lib.ptr(state), _lib.ptr(o), _lib.is_bf16(o),
                  _lib.stream_of(q), tag="kalman_step")
    return o, precision_out


def kdn_gemv(x, weight, bias=None, *, gated=False):
    """``F.linear(x, weight, bias)`` for at most 8 rows through the weight-streaming ``kdn_gemv``:
    bf16 ``weight`` [N,K] (K % 8 == 0), bf16 ``bias`` or None, ``x`` [..., K] bf16 or fp32;
    fp32 accumulation, output in x's dtype.  ``gated=True`` takes a packed ``weight`` [2N,K] =
    [w1; w2] (bias [2N]) and returns the SwiGLU gate silu(x w1^T + b1) * (x w2^T + b2), [..., N]."""
    *lead, K = x.shape
    R = weight.shape[0]
    if weight.dtype != torch.bfloat16 or weight.shape != (R, K) or not weight.is_contiguous() or K % 8:
        raise ValueError("kdn_gemv needs a contiguous bf16 weight [N, K] with K % 8 == 0")
    if gated and R % 2:
        raise ValueError(f"a gated kdn_gemv takes a packed [2N, K] weight, got {R} rows")
    N = R // 2 if gated else R
    if bias is not None and (bias.dtype != torch.bfloat16 or bias.shape != (R,) or not bias.is_contiguous()):
        raise ValueError(f"kdn_gemv takes a contiguous bf16 bias [{R}] or None")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"x must be bf16 or fp32, got {x.dtype}")
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    if M > 8:
        raise ValueError(f"kdn_gemv takes at most 8 rows, got {M}")
    # 16-byte aligned rows; a view of one row keeps its parent's stride and offset (contiguous()
    # returns such a view unchanged), so misaligned inputs are cloned
    if x2.stride(-1) != 1 or x2.data_ptr() % 16 or (M > 1 and (x2.stride(0) * x2.element_size()) % 16):
        x2 = x2.clone(memory_format=torch.contiguous_format)
    row_stride = x2.stride(0) if M > 1 else K
    _lib.require_device(x2, weight, bias)
    y = torch.empty((M, N), device=x.device, dtype=x.dtype)
    if M and N:
        with torch.cuda.device(x.device):
            _lib.call("kdn_gemv", _lib.ptr(x2), _lib.is_bf16(x2), row_stride, _lib.ptr(weight), _lib.ptr(bias), M, N, K,
                      int(bool(gated)), _lib.ptr(y), y.stride(0), _lib.stream_of(x2))
    return y.view(*lead, N)


__all__ = ("kdn_memory_step", "kdn_kalman_step", "kdn_gemv")
