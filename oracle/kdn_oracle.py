"""CPU restatement of the Kalman Delta Network recurrences (TEST INFRASTRUCTURE ONLY).

This module is the parity checker for the HIP implementation in
``kalman-delta-networks_amd``.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product path never does.

Everything here is plain PyTorch on the CPU, computed in fp64 when any input is
fp64 and in fp32 otherwise, and differentiable with torch autograd (the HIP
backward is checked against autograd of these functions).

What each function restates (reference = ngocbh/kalman-delta-networks):

* ``iso_gain_tokenwise``     -- lit_gpt/kdn_ops/iso_kdn_naive.py:200-251
* ``diag_gain_tokenwise``    -- lit_gpt/kdn_ops/diag_kdn_naive.py:217-276
* ``memory_tokenwise``       -- iso_kdn_naive.py:308-332, diag_kdn_naive.py:479-500
* ``iso_recurrent``          -- iso_kdn_naive.py:376-440
* ``diag_recurrent``         -- diag_kdn_naive.py:503-567
* ``iso_gain_mobius`` / ``diag_gain_mobius`` -- the Mobius chunk forms of
  iso_kdn_naive.py:590-634 and diag_kdn_naive.py:285-369 (second, independent form)
* ``memory_chunked_wy``      -- the WY chunk form of iso_kdn_naive.py:449-533 and
  diag_kdn_naive.py:570-655 (second, independent form)
* ``iso_gate_frontend``      -- iso_kdn_chunk.py:787-813 (gate/a/omega/r/mu maps)
* ``diag_frontend``          -- diag_kdn_chunk.py:1885-1905 (alpha clamp, omega, r, mu)
* ``iso_gain_unit_key``      -- the production unit-key iso gain (iso_kdn_chunk.py:1496-1518,
  1586-1594), evaluated through ``iso_gain_tokenwise`` itself on a one-channel problem, so it is
  pinned by the golden vectors of the tokenwise gain; a CPU test also checks it against the
  closed form z/(r+z), p' = r z/(r + s z) and against the tokenwise gain on random unit keys.
* ``diag_normalize``         -- diag_kdn_chunk.py:194-232 (x / max(||x||, 1e-12)); pinned
  against torch.nn.functional.normalize (a library routine with the same definition).
* ``l2norm_fla``             -- FLA l2norm_fwd used at iso_kdn_chunk.py:2203-2204
  (flash-linear-attention @ 4b02d15d; x * rsqrt(sum x^2 + 1e-6)).  FLA is not vendored in
  the reference, so no golden vector covers it; it is pinned by its properties (unit norm,
  zero row, scale invariance, and the eps inside the square root at |x|^2 = eps).
* ``iso_mixer`` / ``diag_mixer`` -- the composition order of iso_kdn.py:277-304 and
  diag_kdn.py:315-345 (frontend -> gain -> memory scan).
* ``short_conv_silu``        -- fixed-length causal depthwise convolution (width 4, no bias)
  + SiLU: FLA causal_conv1d as called at diag_kdn.py:75-96 and per q|k|v group by
  iso_kdn_chunk.py:56-120 (packed forward kernel).  Pinned against torch's conv1d
  (``short_conv_silu_conv1d``, a library routine) and brute force; FLA's own rounding points
  are not in the reference tree (PARITY UNPINNED beyond the f32-then-round convention).
* ``qkv_conv_backward``      -- the reference's packed backward kernel rule,
  iso_kdn_chunk.py:127-254 + 379-437 (preactivation recomputed into x's dtype, then
  g = dy s (1 + y (1 - s)); dx and dw sums); pinned by autograd of ``short_conv_silu`` (exact
  when the preactivation is not rounded).
* ``rms_norm_gated``         -- FLA FusedRMSNormGated(activation="sigmoid"|"swish") as the
  layers' o_norm (iso_kdn.py:192-196,305-312; diag_kdn.py:216-219,346):
  x rsqrt(mean x^2 + eps) w act(g).  FLA is not vendored: PARITY UNPINNED beyond this formula.
* ``rms_norm``               -- the model's FusedRMSNorm (rmsnorm.py:1141-1216, LayerNormFn with
  is_rms_norm, no residual): pinned against torch's F.rms_norm (a library routine).
* ``linear`` / ``amp_round`` / ``swiglu`` -- F.linear and SwiGLU (model.py:452-464), with the bf16
  rounding points of CUDA bf16 autocast when ``amp``; swiglu pinned by a closed form.
* ``iso_layer`` / ``diag_layer`` -- the layer compositions of iso_kdn.py:262-314 and
  diag_kdn.py:259-357 (projection slices, convolutions, mixer, gated norm, output projection);
  ``gpt_forward`` -- GPT/Block of model.py:95-162,217-298.  Pinned by the reference's own
  parameter totals (the modules' shapes), closed-form reductions (zero output projections make
  every block the identity plus its MLP; zero MLP and mixer outputs leave
  lm_head(ln_f(wte[idx]))), and the mixer composition's own pins above.  Which projection slice
  feeds which operand is a restatement of the layer files: PARTIALLY PINNED.

How each is pinned (see tests/test_oracle_*.py):
  golden vectors written from the reference's own oracle files
  (tests/golden/make_golden.py); tokenwise vs Mobius/WY chunk forms (independent
  decompositions); closed forms (T=1, alpha=1 plain delta rule, kappa=0 pure decay,
  scalar Kalman filter for K=1); gradcheck in fp64.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F

LOG2E = 1.4426950408889634


def _dtype(*xs) -> torch.dtype:
    return torch.float64 if any(isinstance(x, torch.Tensor) and x.dtype == torch.float64 for x in xs) else torch.float32


def _bcast_precision_iso(p, B: int, H: int, dtype) -> torch.Tensor:
    if not isinstance(p, torch.Tensor):
        return torch.full((B, H), float(p), dtype=dtype)
    p = p.to(dtype)
    if p.ndim == 0:
        return p.expand(B, H)
    if p.shape == (H,):
        return p.view(1, H).expand(B, H)
    if p.shape == (B, H):
        return p
    raise ValueError(f"initial_precision must be scalar, [H] or [B,H]; got {tuple(p.shape)}")


def _bcast_precision_diag(p, B: int, H: int, K: int, dtype) -> torch.Tensor:
    if not isinstance(p, torch.Tensor):
        return torch.full((B, H, K), float(p), dtype=dtype)
    p = p.to(dtype)
    if p.ndim == 0:
        return p.expand(B, H, K)
    if p.shape == (H,):
        return p.view(1, H, 1).expand(B, H, K)
    if p.shape == (B, H):
        return p.view(B, H, 1).expand(B, H, K)
    if p.shape == (B, H, K):
        return p
    raise ValueError(f"initial_precision must be scalar, [H], [B,H] or [B,H,K]; got {tuple(p.shape)}")


def _info_scale(s, H: int, K: int, dtype) -> torch.Tensor:
    if s is None:
        return torch.full((H,), float(K), dtype=dtype)
    if isinstance(s, torch.Tensor):
        return s.to(dtype).expand(H) if s.ndim == 0 else s.to(dtype)
    return torch.full((H,), float(s), dtype=dtype)


# ----------------------------------------------------------------------------
# Uncertainty (gain) recurrences, tokenwise.
# ----------------------------------------------------------------------------

def iso_gain_tokenwise(k, alpha, omega, r, *, info_scale=None, initial_precision=1.0,
                       output_final_state=False):
    """Scalar-precision Kalman gain, one token at a time (iso_kdn_naive.py:200-251).

    a_t = mean_i alpha_ti^2; z_t = a_t / c_{t-1} + omega_t;
    beta_t = z_t / (r_t + z_t |k_t|^2); c_t = 1/z_t + s |k_t|^2 / (K r_t).
    """
    dt = _dtype(k, alpha, omega, r, initial_precision, info_scale)
    B, T, H, K = k.shape
    k, alpha, omega, r = (x.to(dt) for x in (k, alpha, omega, r))
    c = _bcast_precision_iso(initial_precision, B, H, dt)
    s = _info_scale(info_scale, H, K, dt).view(1, H) / K
    contraction = alpha.square().mean(-1)
    knorm2 = k.square().sum(-1)
    betas = []
    for t in range(T):
        z = contraction[:, t] / c + omega[:, t]
        betas.append(z / (r[:, t] + z * knorm2[:, t]))
        c = 1.0 / z + s * knorm2[:, t] / r[:, t]
    beta = torch.stack(betas, 1) if T else k.sum(-1) * 0
    return beta, (c if output_final_state else None)


def diag_gain_tokenwise(k, alpha, omega, r, *, info_scale=None, initial_precision=1.0,
                        output_final_state=False):
    """Per-channel covariance Kalman gain (diag_kdn_naive.py:217-276).

    p_hat = alpha^2 p + omega; kappa = p_hat k / (r + sum_i p_hat_i k_i^2);
    p = p_hat / (1 + s k^2 / r * p_hat)   (no division by K here).
    """
    dt = _dtype(k, alpha, omega, r, initial_precision, info_scale)
    B, T, H, K = k.shape
    k, alpha, omega, r = (x.to(dt) for x in (k, alpha, omega, r))
    p = 1.0 / _bcast_precision_diag(initial_precision, B, H, K, dt)
    s = _info_scale(info_scale, H, K, dt).view(1, H, 1)
    gains = []
    for t in range(T):
        ph = alpha[:, t].square() * p + omega[:, t]
        kt = k[:, t]
        den = r[:, t, :, None] + (ph * kt.square()).sum(-1, keepdim=True)
        gains.append(ph * kt / den)
        p = ph / (1.0 + s * kt.square() / r[:, t, :, None] * ph)
    kappa = torch.stack(gains, 1) if T else k * 0
    return kappa, ((1.0 / p) if output_final_state else None)


def iso_gain_unit_key(a, omega, r, initial_precision, *, posterior_scale=1.0, output_final_state=False):
    """The production iso gain (iso_kdn_chunk.py:1496-1518,1586-1594): the scalars a = mean_i alpha_i^2,
    omega, r [B,T,H] with |k| = 1, s = info_scale / head_dim = ``posterior_scale``.

    Evaluated as ``iso_gain_tokenwise`` itself (golden-pinned) on a one-channel problem with the
    same a, omega, r: k = 1 and alpha = sqrt(a) give mean alpha^2 = a and |k|^2 = 1, and
    info_scale = s (the one-channel s / K).  So z = a / c + omega, beta = z / (r + z),
    c' = 1 / z + s / r -- the unit-key form the kernels implement.  Returns (beta, c_T or None)."""
    one = torch.ones_like(a)[..., None]
    beta, c = iso_gain_tokenwise(one, a.sqrt()[..., None], omega, r, info_scale=posterior_scale,
                                 initial_precision=initial_precision, output_final_state=output_final_state)
    return beta, c


# ----------------------------------------------------------------------------
# Uncertainty recurrences as chunked Mobius-map compositions (second form).
# ----------------------------------------------------------------------------

def _mobius(m, p):
    return (m[..., 0, 0] * p + m[..., 0, 1]) / (m[..., 1, 0] * p + m[..., 1, 1])


def iso_gain_mobius(k, alpha, omega, r, *, info_scale=None, initial_precision=1.0,
                    chunk_size=64, output_final_state=False):
    """Covariance p = 1/c advanced by 2x2 projective maps composed per chunk.

    Token map acting on p: p' = (r a p + r w) / (s' a p + r + s' w) with
    s' = s |k|^2 / K, i.e. [[r a, r w], [s' a, r + s' w]] (iso_kdn_naive.py:608-632).
    """
    dt = _dtype(k, alpha, omega, r, initial_precision, info_scale)
    B, T, H, K = k.shape
    k, alpha, omega, r = (x.to(dt) for x in (k, alpha, omega, r))
    p0 = 1.0 / _bcast_precision_iso(initial_precision, B, H, dt)
    s = _info_scale(info_scale, H, K, dt).view(1, H) / K
    a = alpha.square().mean(-1)
    n2 = k.square().sum(-1)
    out = []
    for c0 in range(0, T, chunk_size):
        m = torch.eye(2, dtype=dt).expand(B, H, 2, 2)
        for t in range(c0, min(T, c0 + chunk_size)):
            p = _mobius(m, p0)
            z = a[:, t] * p + omega[:, t]
            out.append(z / (r[:, t] + z * n2[:, t]))
            sw = s * n2[:, t]
            tm = torch.stack((torch.stack((r[:, t] * a[:, t], r[:, t] * omega[:, t]), -1),
                              torch.stack((sw * a[:, t], r[:, t] + sw * omega[:, t]), -1)), -2)
            m = tm @ m
            m = m / m.abs().amax((-2, -1), keepdim=True)
        p0 = _mobius(m, p0)
    beta = torch.stack(out, 1) if T else k.sum(-1) * 0
    return beta, ((1.0 / p0) if output_final_state else None)


def diag_gain_mobius(k, alpha, omega, r, *, info_scale=None, initial_precision=1.0,
                     chunk_size=32, output_final_state=False):
    """Per-channel map [[a^2, w], [u a^2, 1 + u w]], u = s k^2 / r (diag_kdn_naive.py:338-360)."""
    dt = _dtype(k, alpha, omega, r, initial_precision, info_scale)
    B, T, H, K = k.shape
    k, alpha, omega, r = (x.to(dt) for x in (k, alpha, omega, r))
    p0 = 1.0 / _bcast_precision_diag(initial_precision, B, H, K, dt)
    s = _info_scale(info_scale, H, K, dt).view(1, H, 1)
    out = []
    for c0 in range(0, T, chunk_size):
        m = torch.eye(2, dtype=dt).expand(B, H, K, 2, 2)
        for t in range(c0, min(T, c0 + chunk_size)):
            p = _mobius(m, p0)
            a2 = alpha[:, t].square()
            ph = a2 * p + omega[:, t]
            kt = k[:, t]
            den = r[:, t, :, None] + (ph * kt.square()).sum(-1, keepdim=True)
            out.append(ph * kt / den)
            u = s * kt.square() / r[:, t, :, None]
            tm = torch.stack((torch.stack((a2, omega[:, t]), -1),
                              torch.stack((u * a2, 1.0 + u * omega[:, t]), -1)), -2)
            m = tm @ m
            m = m / m.abs().amax((-2, -1), keepdim=True)
        p0 = _mobius(m, p0)
    kappa = torch.stack(out, 1) if T else k * 0
    return kappa, ((1.0 / p0) if output_final_state else None)


# ----------------------------------------------------------------------------
# Memory recurrence (shared by both variants; kappa = beta k for iso).
# ----------------------------------------------------------------------------

def memory_tokenwise(q, k, v, alpha, kappa, *, scale, initial_state=None):
    """S_hat = alpha (.) S; delta = v - k^T S_hat; S = S_hat + kappa delta^T; o = scale q^T S.

    (iso_kdn_naive.py:308-332, diag_kdn_naive.py:479-500.)  Shapes: q,k,alpha,kappa
    [B,T,H,K], v [B,T,H,V]; returns o [B,T,H,V] and S [B,H,K,V].
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    S = torch.zeros(B, H, K, V, dtype=q.dtype) if initial_state is None else initial_state.to(q.dtype)
    outs = []
    for t in range(T):
        Sh = alpha[:, t, :, :, None] * S
        delta = v[:, t] - torch.einsum("bhk,bhkv->bhv", k[:, t], Sh)
        S = Sh + kappa[:, t, :, :, None] * delta[:, :, None, :]
        outs.append(scale * torch.einsum("bhk,bhkv->bhv", q[:, t], S))
    o = torch.stack(outs, 1) if T else v * 0
    return o, S


def memory_chunked_wy(q, k, v, alpha, kappa, *, scale, initial_state=None, chunk_size=64):
    """Chunked WY form of the same recurrence (second, independent decomposition).

    Within a chunk with G = cumsum(log alpha):
      N[c,s] = sum_i k_ci exp(G_ci - G_si) kappa_si (s < c);  A = (I + N)^-1
      U = A V, W = A (K e^G), D = U - W S
      O = scale (Q e^G) S + scale tril(Q Gamma kappa^T) D
      S' = e^{G_last} S + (e^{G_last - G} kappa)^T D
    (iso_kdn_naive.py:449-533, diag_kdn_naive.py:570-655.)
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    S = torch.zeros(B, H, K, V, dtype=q.dtype) if initial_state is None else initial_state.to(q.dtype)
    outs = []
    for c0 in range(0, T, chunk_size):
        c1 = min(T, c0 + chunk_size)
        L = c1 - c0
        qc = q[:, c0:c1].transpose(1, 2)
        kc = k[:, c0:c1].transpose(1, 2)
        vc = v[:, c0:c1].transpose(1, 2)
        kap = kappa[:, c0:c1].transpose(1, 2)
        G = alpha[:, c0:c1].log().transpose(1, 2).cumsum(2)
        diff = G[:, :, :, None, :] - G[:, :, None, :, :]            # [B,H,c,s,K]
        low = torch.tril(torch.ones(L, L, dtype=torch.bool), -1)
        lowd = torch.tril(torch.ones(L, L, dtype=torch.bool), 0)
        E = torch.where(lowd[:, :, None], diff, torch.zeros((), dtype=q.dtype)).exp()
        N = torch.einsum("bhck,bhcsk,bhsk->bhcs", kc, E, kap) * low
        Mq = torch.einsum("bhck,bhcsk,bhsk->bhcs", qc, E, kap) * lowd
        I = torch.eye(L, dtype=q.dtype)
        U = torch.linalg.solve_triangular(I + N, vc, upper=False, unitriangular=True)
        W = torch.linalg.solve_triangular(I + N, kc * G.exp(), upper=False, unitriangular=True)
        D = U - W @ S
        outs.append((scale * ((qc * G.exp()) @ S + Mq @ D)).transpose(1, 2))
        Gl = G[:, :, -1:, :]
        S = Gl[:, :, 0, :, None].exp() * S + ((Gl - G).exp() * kap).transpose(-1, -2) @ D
    o = torch.cat(outs, 1) if T else v * 0
    return o, S


def iso_recurrent(q, k, v, alpha, omega, r, *, info_scale=None, scale=None, initial_state=None,
                  initial_precision=1.0, output_final_state=False, chunked=False, chunk_size=64):
    """Full iso recurrence (iso_kdn_naive.py:376-440); q,k used exactly as given."""
    dt = _dtype(q, k, v, alpha, omega, r, initial_state, initial_precision, info_scale)
    q, k, v, alpha, omega, r = (x.to(dt) for x in (q, k, v, alpha, omega, r))
    K = q.shape[-1]
    scale = K ** -0.5 if scale is None else float(scale)
    gain = iso_gain_mobius if chunked else iso_gain_tokenwise
    kw = dict(chunk_size=chunk_size) if chunked else {}
    beta, prec = gain(k, alpha, omega, r, info_scale=info_scale, initial_precision=initial_precision,
                      output_final_state=True, **kw)
    mem = memory_chunked_wy if chunked else memory_tokenwise
    o, S = mem(q, k, v, alpha, beta[..., None] * k, scale=scale, initial_state=initial_state, **kw)
    return o, ((S, prec) if output_final_state else None)


def diag_recurrent(q, k, v, alpha, omega, r, *, info_scale=None, scale=None, initial_state=None,
                   initial_precision=1.0, output_final_state=False, chunked=False, chunk_size=32):
    """Full diag recurrence (diag_kdn_naive.py:503-567); q,k used exactly as given."""
    dt = _dtype(q, k, v, alpha, omega, r, initial_state, initial_precision, info_scale)
    q, k, v, alpha, omega, r = (x.to(dt) for x in (q, k, v, alpha, omega, r))
    K = q.shape[-1]
    scale = K ** -0.5 if scale is None else float(scale)
    gain = diag_gain_mobius if chunked else diag_gain_tokenwise
    kw = dict(chunk_size=chunk_size) if chunked else {}
    kappa, prec = gain(k, alpha, omega, r, info_scale=info_scale, initial_precision=initial_precision,
                       output_final_state=True, **kw)
    mem = memory_chunked_wy if chunked else memory_tokenwise
    o, S = mem(q, k, v, alpha, kappa, scale=scale, initial_state=initial_state, **kw)
    return o, ((S, prec) if output_final_state else None)


# ----------------------------------------------------------------------------
# Production frontends (elementwise maps restated from the kernel sources).
# ----------------------------------------------------------------------------

def softplus(x):
    """torch softplus (threshold 20), the convention used throughout."""
    return F.softplus(x)


def _w(x):
    """Working precision: fp64 stays fp64, anything else computes in fp32."""
    return x if x.dtype == torch.float64 else x.float()


def l2norm_fla(x, eps: float = 1e-6):
    """x * rsqrt(sum x^2 + eps) over the last dim (FLA l2norm_fwd, flash-linear-attention @ 4b02d15d,
    as called at iso_kdn_chunk.py:2203-2204).  Pinned by its properties: unit norm when
    sum x^2 >> eps, a zero row maps to zero, invariance to positive scaling of large rows, and the
    eps inside the square root (x = c e_1 with c^2 = eps maps to 1/sqrt(2) e_1)."""
    return x * torch.rsqrt(x.square().sum(-1, keepdim=True) + eps)


def diag_normalize(x):
    """x / max(||x||_2, 1e-12) over the last dim (diag_kdn_chunk.py:194-232)."""
    return x / x.norm(dim=-1, keepdim=True).clamp_min(1e-12)


def chunk_local_prefix(x, chunk: int):
    """Inclusive cumulative sum over time that restarts every ``chunk`` tokens ([B,T,...])."""
    T = x.shape[1]
    parts = [x[:, c0:c0 + chunk].cumsum(1) for c0 in range(0, T, chunk)]
    return torch.cat(parts, 1) if parts else x


def iso_gate_frontend(g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias, mu_param,
                      omega_min=0.0, r_min=0.01, chunk=64):
    """iso_kdn_chunk.py:787-813.

    g = -exp(A_log) softplus(g_raw + dt_bias) (per channel, natural log of alpha);
    g_cumsum = chunk-local inclusive prefix of g times log2(e);
    a = mean_K exp(2 g); omega = omega_min + softplus(raw + b); r = r_min + softplus(raw + b);
    mu = 0.1 + softplus(mu_param).  Returns (g_log, g_cumsum_base2, a, omega, r, mu).
    """
    B, T, H, K = g_raw.shape
    x = _w(g_raw) + _w(dt_bias).view(H, K)
    g = -_w(A_log).exp().view(H, 1) * softplus(x)
    gc = chunk_local_prefix(g, chunk) * LOG2E
    a = (2.0 * g).exp().mean(-1)
    orr = _w(omega_r_raw)
    omega = omega_min + softplus(orr[..., :H] + _w(omega_bias))
    r = r_min + softplus(orr[..., H:] + _w(r_bias))
    mu = 0.1 + softplus(_w(mu_param))
    return g, gc, a, omega, r, mu


def diag_frontend(retention_raw, omega_raw, r_raw, A_log, dt_bias, mu_param, chunk=32):
    """diag_kdn_chunk.py:1885-1905.

    alpha = exp(-exp(A_log) softplus(f + dt_bias)); the memory path uses
    l = log(max(alpha, 1e-6)) and its chunk-local base-2 prefix; omega = softplus(z);
    r = 0.01 + softplus(y); mu = 0.1 + softplus(mu_param).
    Returns (l_mem, g_cumsum_base2, alpha, omega, r, mu).
    """
    B, T, H, K = retention_raw.shape
    x = _w(retention_raw) + _w(dt_bias).view(H, K)
    ell = -_w(A_log).exp().view(H, 1) * softplus(x)
    alpha = ell.exp()
    # memory path: log(max(alpha, 1e-6)), i.e. ell itself unless alpha is below the floor
    l_mem = torch.where(alpha >= 1e-6, ell, torch.full_like(ell, math.log(1e-6)))
    gc = chunk_local_prefix(l_mem, chunk) * LOG2E
    omega = softplus(_w(omega_raw))
    r = 0.01 + softplus(_w(r_raw))
    mu = 0.1 + softplus(_w(mu_param))
    return l_mem, gc, alpha, omega, r, mu


# ----------------------------------------------------------------------------
# Composed mixers at the kdn_ops boundary (frontend -> gain -> memory), fp32 CPU.
# ----------------------------------------------------------------------------

def iso_mixer(q_raw, k_raw, v, g_raw, omega_r_raw, omega_bias, r_bias, A_log, dt_bias, mu_param,
              *, omega_min=0.0, r_min=0.01, info_scale=None, scale=None, chunked=False, round_qk=False):
    """iso_kdn.py:277-304: gate frontend, scalar gain on unit keys, KDA memory scan.

    The production gain consumes (a, omega, r, mu) only and assumes |k| = 1
    (iso_kdn_chunk.py:1586-1594); the memory scan L2-normalises q and k inside
    (iso_kdn_chunk.py:2203-2204) and uses alpha = exp(g) per channel.  ``round_qk`` models
    bf16 inputs: FLA's l2norm_fwd writes its output in the input's dtype, so the production scan
    consumes the normalised q, k rounded to bf16 (and their cotangents come back in bf16).
    """
    K = q_raw.shape[-1]
    g, _gc, a, omega, r, mu = iso_gate_frontend(g_raw, omega_r_raw, omega_bias, r_bias, A_log,
                                                dt_bias, mu_param, omega_min, r_min)
    qn = amp_round(l2norm_fla(_w(q_raw)), round_qk)
    kn = amp_round(l2norm_fla(_w(k_raw)), round_qk)
    alpha = g.exp()
    # Gain on the production scalars (unit-norm keys): beta = z / (r + z)
    s = (float(K) if info_scale is None else float(info_scale)) / K
    beta, _ = iso_gain_unit_key(a, omega, r, mu, posterior_scale=s)
    sc = K ** -0.5 if scale is None else scale
    mem = memory_chunked_wy if chunked else memory_tokenwise
    o, _ = mem(qn, kn, _w(v), alpha, beta[..., None] * kn, scale=sc)
    return o


def diag_mixer(q_raw, k_raw, v, retention_raw, omega_raw, r_raw, A_log, dt_bias, mu_param,
               *, scale=None, chunked=False, initial_state=None, initial_precision=None,
               output_final_state=False, gain_chunked=None, round_qk=True):
    """diag_kdn.py:315-345: normalise, frontend, vector gain, memory scan (fp32 output).

    The memory path consumes alpha clamped at 1e-6 (through g_cumsum) while the
    gain consumes the unclamped alpha (diag_kdn_chunk.py:1887-1898).  ``chunked`` selects the WY
    chunk form of the memory and (unless ``gain_chunked`` says otherwise) the Mobius form of the
    gain; the forms agree to rounding (tokenwise == chunked is pinned on the CPU).  ``round_qk``
    (default on, as in production) models the normalisation's bf16 memory operands: q_memory and
    k_memory are bf16 while the gain's k is fp32 (diag_kdn_chunk.py:2045-2076), cotangents included.
    """
    K = q_raw.shape[-1]
    qn = diag_normalize(_w(q_raw))
    kn = diag_normalize(_w(k_raw))
    l_mem, _gc, alpha, omega, r, mu = diag_frontend(retention_raw, omega_raw, r_raw, A_log, dt_bias, mu_param)
    prec = mu if initial_precision is None else initial_precision
    gain = diag_gain_mobius if (chunked if gain_chunked is None else gain_chunked) else diag_gain_tokenwise
    kappa, fprec = gain(kn, alpha, omega, r, info_scale=float(K), initial_precision=prec,
                        output_final_state=True)
    sc = K ** -0.5 if scale is None else scale
    mem = memory_chunked_wy if chunked else memory_tokenwise
    o, S = mem(amp_round(qn, round_qk), amp_round(kn, round_qk), _w(v), l_mem.exp(), kappa, scale=sc,
               initial_state=initial_state)
    if output_final_state:
        return o, (S, fprec)
    return o


# ----------------------------------------------------------------------------
# Layer frontends around the scan (short convolution, gated output norm).
# ----------------------------------------------------------------------------

SHORT_CONV_WIDTH = 4


def short_conv_silu(x, weight):
    """silu(sum_j w[d, j] x[t - 3 + j, d]) with zero history; x [B,T,D], weight [D,4]."""
    xw, ww = _w(x), _w(weight)
    B, T, D = xw.shape
    W = ww.shape[1]
    pad = torch.cat([xw.new_zeros(B, W - 1, D), xw], 1)
    y = sum(pad[:, j:j + T] * ww[:, j] for j in range(W))
    return F.silu(y)


def short_conv_silu_conv1d(x, weight):
    """The same map through torch's grouped conv1d (independent formulation)."""
    xw, ww = _w(x), _w(weight)
    T, D = xw.shape[1], xw.shape[2]
    y = F.conv1d(xw.transpose(1, 2), ww[:, None, :], padding=ww.shape[1] - 1, groups=D)[..., :T]
    return F.silu(y.transpose(1, 2))


def qkv_conv_backward(x, weight, dy, raw_dtype=None):
    """Gradients of one convolution group by the reference kernel's rule: the preactivation is
    recomputed and (for ``raw_dtype`` bf16) rounded as its raw_y buffer is, then
    g = dy * s * (1 + y (1 - s)), dx[t] = sum_j w[j] g[t + 3 - j], dw[j] = sum_{b,t} g[t] x[t - 3 + j]."""
    xw, ww, dyw = _w(x), _w(weight), _w(dy)
    B, T, D = xw.shape
    W = ww.shape[1]
    pad = torch.cat([xw.new_zeros(B, W - 1, D), xw], 1)
    y = sum(pad[:, j:j + T] * ww[:, j] for j in range(W))
    if raw_dtype is not None:
        y = y.to(raw_dtype).to(y.dtype)
    s = torch.sigmoid(y)
    g = dyw * s * (1 + y * (1 - s))
    gpad = torch.cat([g, g.new_zeros(B, W - 1, D)], 1)
    dx = sum(gpad[:, W - 1 - j:W - 1 - j + T] * ww[:, j] for j in range(W))
    dw = torch.stack([(g * pad[:, j:j + T]).sum((0, 1)) for j in range(W)], -1)
    return dx, dw


def rms_norm_gated(x, g, weight, eps: float = 1e-5, activation: str = "sigmoid"):
    """x * rsqrt(mean(x^2) + eps) * weight * act(g) over the last dim; act = sigmoid or swish."""
    xw, gw, ww = _w(x), _w(g), _w(weight)
    n = xw * torch.rsqrt(xw.square().mean(-1, keepdim=True) + eps)
    a = torch.sigmoid(gw) if activation == "sigmoid" else gw * torch.sigmoid(gw)
    return n * ww * a


# ----------------------------------------------------------------------------
# The config-4 block stack: layers, block, GPT (compositions of the above).
# ----------------------------------------------------------------------------

def rms_norm(x, weight, eps: float = 1e-5):
    """FusedRMSNorm without residual/dropout (rmsnorm.py:1141-1216): x rsqrt(mean x^2 + eps) w."""
    xw = _w(x)
    return xw * torch.rsqrt(xw.square().mean(-1, keepdim=True) + eps) * _w(weight)


class _Bf16Round(torch.autograd.Function):
    """Rounds to bf16 in the forward and rounds the cotangent to bf16 in the backward: a tensor that
    autocast stores in bf16 also receives its gradient in bf16."""

    @staticmethod
    def forward(ctx, x):
        return x.to(torch.bfloat16).to(x.dtype)

    @staticmethod
    def backward(ctx, g):
        return g.to(torch.bfloat16).to(g.dtype)


def amp_round(x, amp: bool):
    """Round to bf16 where CUDA bf16 autocast stores a bf16 tensor (identity otherwise); the
    backward rounds that tensor's cotangent to bf16 as well, as autograd does for a bf16 tensor."""
    return _Bf16Round.apply(x) if amp else x


def linear(x, weight, bias=None, amp: bool = False):
    """F.linear; under bf16 autocast its operands and its result are bf16 (f32 accumulation)."""
    x, weight = amp_round(x, amp), amp_round(_w(weight), amp)
    y = x @ weight.transpose(0, 1)
    if bias is not None:
        y = y + amp_round(_w(bias), amp)
    return amp_round(y, amp)


def swiglu(x, w1, w2, w3, amp: bool = False):
    """model.py:452-464: w3(silu(w1 x) * w2 x)."""
    a, b = linear(x, w1, amp=amp), linear(x, w2, amp=amp)
    return linear(amp_round(amp_round(F.silu(a), amp) * b, amp), w3, amp=amp)


def iso_layer(p, x, *, eps=1e-5, omega_min=0.0, r_min=0.01, info_scale=None, amp=False, chunked=False,
              scan_bf16=False):
    """IsotropicKalmanDeltaNetwork.forward (iso_kdn.py:262-314) on a state dict ``p`` of the
    layer (reference parameter names): packed q|k|v projection + per-group SiLU short
    convolution; [f0 | omega | r] packed projection, f_proj[1] on the f0 slice; iso_mixer;
    sigmoid-gated RMS norm against g_proj(x); o_proj.  ``chunked`` runs the mixer's memory in the
    WY chunk form (equal to the tokenwise form to rounding; faster at long T).  ``scan_bf16`` rounds
    the normalised q, k and v to bf16 at the memory scan's boundary, for a model whose scan takes bf16
    operands from fp32 inputs (the HIP scan does; under autocast, ``amp``, they are bf16 already)."""
    H = p["A_log"].shape[0]
    Dm = p["qkv_pack.projection_weight"].shape[0] // 3
    K = Dm // H
    B, T, _ = x.shape
    qkv = linear(x, p["qkv_pack.projection_weight"], amp=amp)
    cw = p["qkv_pack.convolution_weight"]
    q, k, v = (amp_round(short_conv_silu(qkv[..., i * Dm:(i + 1) * Dm], cw[i * Dm:(i + 1) * Dm]), amp)
               for i in range(3))
    packed = linear(x, p["f_omega_r_proj.weight"], amp=amp)
    f_hidden, omega_r_raw = packed[..., :K], packed[..., K:]
    g_raw = linear(f_hidden, p["f_proj.1.weight"], amp=amp)
    v = amp_round(v, scan_bf16)
    o = iso_mixer(q.view(B, T, H, K), k.view(B, T, H, K), v.view(B, T, H, K), g_raw.view(B, T, H, K),
                  omega_r_raw, p["omega_proj.bias"], p["r_proj.bias"], p["A_log"], p["dt_bias"],
                  p["initial_precision_param"], omega_min=omega_min, r_min=r_min, info_scale=info_scale,
                  round_qk=amp or scan_bf16, chunked=chunked)
    o = amp_round(o, amp)
    gate = linear(linear(x, p["g_proj.0.weight"], amp=amp), p["g_proj.1.weight"], p["g_proj.1.bias"], amp=amp)
    y = amp_round(rms_norm_gated(o, gate.view(B, T, H, K), p["o_norm.weight"], eps, "sigmoid"), amp)
    return linear(y.reshape(B, T, Dm), p["o_proj.weight"], amp=amp)


def diag_layer(p, x, *, eps=1e-5, amp=False):
    """DiagonalKalmanDeltaNetwork.forward (diag_kdn.py:259-357) on a state dict ``p`` of the layer:
    q/k/v projections + SiLU short convolutions, f_proj / omega_proj two-layer projections,
    r_proj, diag_mixer (its f32 output stored at v's dtype), gated RMS norm, o_proj."""
    H = p["A_log"].shape[0]
    Dm = p["q_proj.weight"].shape[0]
    K = Dm // H
    B, T, _ = x.shape

    def conv(name):
        y = short_conv_silu(linear(x, p[f"{name}_proj.weight"], amp=amp), p[f"{name}_conv1d.weight"][:, 0, :])
        return amp_round(y, amp).view(B, T, H, K)

    q, k, v = conv("q"), conv("k"), conv("v")
    retention_raw = linear(linear(x, p["f_proj.0.weight"], amp=amp), p["f_proj.1.weight"], amp=amp)
    omega_raw = linear(linear(x, p["omega_proj.0.weight"], amp=amp), p["omega_proj.1.weight"],
                       p["omega_proj.1.bias"], amp=amp)
    r_raw = linear(x, p["r_proj.weight"], p["r_proj.bias"], amp=amp)
    o = diag_mixer(q, k, v, retention_raw.view(B, T, H, K), omega_raw.view(B, T, H, K), r_raw, p["A_log"],
                   p["dt_bias"], p["initial_precision_param"])
    o = amp_round(o, amp)
    gate = linear(linear(x, p["g_proj.0.weight"], amp=amp), p["g_proj.1.weight"], p["g_proj.1.bias"], amp=amp)
    y = amp_round(rms_norm_gated(o, gate.view(B, T, H, K), p["o_norm.weight"], eps, "sigmoid"), amp)
    return linear(y.reshape(B, T, Dm), p["o_proj.weight"], amp=amp)


def _sub(p, prefix):
    return {k[len(prefix):]: v for k, v in p.items() if k.startswith(prefix)}


def gpt_forward(p, idx, *, n_layer, mixer_type, eps=1e-5, amp=False, **mixer_kw):
    """GPT.forward (model.py:95-162) for KDN-only stacks with parallel_residual=False:
    x = wte[idx]; per block x += mixer(norm_1(x)); x += swiglu(norm_2(x)); logits = lm_head(ln_f(x)).
    The residual stream stays in the embedding's dtype (bf16 branch outputs add into f32)."""
    layer = iso_layer if mixer_type == "iso_kdn" else diag_layer
    x = _w(p["transformer.wte.weight"])[idx]
    for i in range(n_layer):
        b = _sub(p, f"transformer.h.{i}.")
        h = layer(_sub(b, "attn."), rms_norm(x, b["norm_1.weight"], eps), eps=eps, amp=amp, **mixer_kw)
        x = x + h
        m = _sub(b, "mlp.swiglu.")
        x = x + swiglu(rms_norm(x, b["norm_2.weight"], eps), m["w1.weight"], m["w2.weight"], m["w3.weight"], amp=amp)
    return linear(rms_norm(x, p["transformer.ln_f.weight"], eps), p["lm_head.weight"], amp=amp)
