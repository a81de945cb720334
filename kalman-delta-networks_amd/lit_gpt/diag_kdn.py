"""Diagonal KDN mixer layer on MI355X (``DiagonalKalmanDeltaNetwork``).

Mirrors ``lit_gpt/diag_kdn.py`` of the reference (ngocbh/kalman-delta-networks): the same
constructor arguments and checks (:101-176), the same parameter names and shapes
(``q_proj``/``k_proj``/``v_proj``, ``q_conv1d.weight`` [D,1,4] and its k/v twins, ``f_proj``,
``A_log``, ``dt_bias``, ``g_proj``, ``o_norm.weight``, ``o_proj``, ``omega_proj`` (a two-layer
projection whose second layer starts at zero), ``r_proj``, ``initial_precision_param``), so a
reference state dict loads, and the same forward composition (:259-357): projections -> SiLU
short convolutions -> q/k normalisation -> per-channel gate frontend -> diagonal Kalman gain ->
chunked memory scan (cast to the value dtype at the store) -> sigmoid-gated RMS norm -> output
projection.  Projections are torch GEMMs; everything else runs in ``libkdn_hip.so``.
The reference's RNG-order-preserving construction is not reproduced (random init differs).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import nn

from ._inference import as_f32, linear, packed_weight, use_packed
from .iso_kdn import _SUPPORTED_HEAD_DIMS, decay_parameters, initial_precision_inverse, validate_training_dtype
from .kdn_ops.diag_kdn_chunk import (_chunk_kalman_as, _diag_kdn_frontend_precumsum_paired, _diag_kdn_normalize,
                                     diag_kdn_front)
from .kdn_ops.gated_norm import FusedRMSNormGated
from .kdn_ops.short_conv import causal_conv1d
from .kdn_ops.step import kdn_kalman_step
from .kdn_state import CONV_TAIL, carry_state, check_state, conv_input_with_tail

_OMEGA_MIN = 0.0
_R_MIN = 0.01


class ShortConvolution(nn.Module):
    """Depthwise width-4 causal convolution + SiLU holding an ``nn.Conv1d``-shaped weight
    [D, 1, 4] (reference diag_kdn.py:65-98)."""

    def __init__(self, hidden_size: int, kernel_size: int = 4):
        super().__init__()
        self.hidden_size = hidden_size
        self.kernel_size = kernel_size
        self.weight = nn.Parameter(torch.empty(hidden_size, 1, kernel_size))
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))

    def forward(self, x):
        y, state = causal_conv1d(x, self.weight.view(self.hidden_size, self.kernel_size), activation="silu")
        if state is not None:
            raise RuntimeError("fixed-length Diagonal KDN convolution returned state")
        return y


class DiagonalKalmanDeltaNetwork(nn.Module):
    """Diagonal KDN mixer (reference diag_kdn.py:101-357), plus an optional carried state."""

    def __init__(self, hidden_size: int = 2304, head_dim: int = 128, num_heads: int = 18, expand_v: float = 1.0,
                 num_v_heads=None, use_short_conv: bool = True, conv_size: int = 4, conv_bias: bool = False,
                 omega_min: float = _OMEGA_MIN, r_min: float = _R_MIN, info_scale=None, norm_eps: float = 1e-5,
                 layer_idx=None):
        if head_dim not in _SUPPORTED_HEAD_DIMS:
            raise ValueError(f"unsupported Diagonal KDN head_dim {head_dim}; expected one of {_SUPPORTED_HEAD_DIMS}")
        if hidden_size != head_dim * num_heads:
            raise ValueError("Diagonal KDN hidden_size must equal head_dim * num_heads; "
                             f"got hidden_size={hidden_size}, head_dim={head_dim}, num_heads={num_heads}")
        if (num_heads if num_v_heads is None else num_v_heads) != num_heads:
            raise ValueError("num_v_heads must equal num_heads for Diagonal KDN")
        if float(expand_v) != 1.0:
            raise ValueError(f"expand_v must be 1.0 for Diagonal KDN, got {expand_v!r}")
        if not use_short_conv or conv_size != 4 or conv_bias:
            raise ValueError("Diagonal KDN requires the biasless width-4 short-convolution path")
        if float(omega_min) != _OMEGA_MIN:
            raise ValueError(f"Diagonal KDN fixes omega_min={_OMEGA_MIN}")
        if float(r_min) != _R_MIN:
            raise ValueError(f"Diagonal KDN fixes r_min={_R_MIN}")
        if info_scale is not None and float(info_scale) != float(head_dim):
            raise ValueError("Diagonal KDN fixes info_scale to the head dimension")
        super().__init__()
        self.hidden_size = hidden_size
        self.expand_v = 1.0
        self.head_dim = self.head_k_dim = self.head_v_dim = head_dim
        self.num_heads = self.num_v_heads = num_heads
        self.key_dim = self.value_dim = self.gate_dim = num_heads * head_dim
        self.layer_idx = layer_idx
        self.omega_min, self.r_min, self.info_scale = _OMEGA_MIN, _R_MIN, float(head_dim)

        self.q_proj = nn.Linear(hidden_size, self.key_dim, bias=False)
        self.k_proj = nn.Linear(hidden_size, self.key_dim, bias=False)
        self.v_proj = nn.Linear(hidden_size, self.value_dim, bias=False)
        self.q_conv1d = ShortConvolution(self.key_dim)
        self.k_conv1d = ShortConvolution(self.key_dim)
        self.v_conv1d = ShortConvolution(self.value_dim)
        self.f_proj = nn.Sequential(nn.Linear(hidden_size, head_dim, bias=False),
                                    nn.Linear(head_dim, self.gate_dim, bias=False))
        self.A_log, self.dt_bias = decay_parameters(num_heads, self.gate_dim)
        self.g_proj = nn.Sequential(nn.Linear(hidden_size, head_dim, bias=False),
                                    nn.Linear(head_dim, self.value_dim, bias=True))
        self.o_norm = FusedRMSNormGated(head_dim, activation="sigmoid", eps=norm_eps)
        self.o_proj = nn.Linear(self.value_dim, hidden_size, bias=False)
        self.omega_proj = nn.Sequential(nn.Linear(hidden_size, head_dim, bias=False),
                                        nn.Linear(head_dim, self.gate_dim, bias=True))
        nn.init.zeros_(self.omega_proj[1].weight)
        nn.init.zeros_(self.omega_proj[1].bias)
        self.omega_proj[1]._kdn_omega_zero = True
        self.r_proj = nn.Linear(hidden_size, num_heads, bias=True)
        self.initial_precision_param = nn.Parameter(torch.full((num_heads,), initial_precision_inverse(),
                                                               dtype=torch.float32))
        self.initial_precision_param._no_weight_decay = True

    def forward(self, hidden_states, attention_mask=None, past_key_values=None, use_cache=False,
                output_attentions=False, **kwargs):
        """Returns ``(output, None, state)``.  Without ``past_key_values`` / ``use_cache`` this is the
        reference's fixed-length forward and ``state`` is None.  With them (state carry, which the
        reference refuses): ``past_key_values`` is the ``KDNLayerState`` after the earlier tokens (None:
        no earlier tokens) and ``use_cache=True`` returns the state after these tokens.  One token
        without autograd runs the single-token step kernel; longer segments run the chunked scan from
        the carried state."""
        requested = tuple(n for n, on in (("attention_mask", attention_mask is not None),
                                          ("output_attentions", output_attentions is not False),
                                          ("kwargs", bool(kwargs))) if on)
        if requested:
            raise ValueError("DiagonalKalmanDeltaNetwork supports only fixed-length sequences (with an optional "
                             f"carried state); unsupported arguments: {requested}")
        if hidden_states.ndim != 3 or hidden_states.shape[-1] != self.hidden_size:
            raise ValueError(f"hidden_states must have shape [B,T,{self.hidden_size}], "
                             f"got {tuple(hidden_states.shape)}")
        if hidden_states.shape[0] == 0 or hidden_states.shape[1] == 0:
            raise ValueError("Diagonal KDN requires non-empty batch and sequence dimensions")
        if torch.is_grad_enabled() and hidden_states.shape[1] < 2:
            raise ValueError("differentiable Diagonal KDN training requires sequence length >= 2; "
                             "the exact one-token convolution update is inference-only")
        if not hidden_states.is_cuda:
            raise ValueError("DiagonalKalmanDeltaNetwork requires CUDA hidden_states")
        validate_training_dtype("Diagonal", training=self.training, hidden_dtype=hidden_states.dtype)
        B, T, _ = hidden_states.shape
        H, K, V = self.num_heads, self.head_k_dim, self.head_v_dim
        stateful = past_key_values is not None or bool(use_cache)
        state = past_key_values
        if state is not None:
            check_state(state, B, H, K, V, 3, (B, H, K), hidden_states.device)
        gate = None
        if use_packed(hidden_states, self):  # a few rows without autograd: the six biasless input GEMMs as one
            D, d = self.key_dim, self.head_k_dim
            w_in = packed_weight(self, "in_proj", (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight,
                                                   self.f_proj[0].weight, self.omega_proj[0].weight,
                                                   self.g_proj[0].weight))
            yq, yk, yv, f_hidden, w_hidden, g_hidden = linear(hidden_states, w_in).split(
                (D, D, self.value_dim, d, d, d), dim=-1)
            projections = (yq, yk, yv)
            retention_raw = linear(f_hidden, self.f_proj[1].weight).view(B, T, H, K)
            omega_raw = linear(w_hidden, self.omega_proj[1].weight, self.omega_proj[1].bias).view(B, T, H, K)
            r_raw = linear(hidden_states, self.r_proj.weight, self.r_proj.bias)  # not packed: its bias rounds with the product
            gate = linear(g_hidden, self.g_proj[1].weight, self.g_proj[1].bias)
        else:
            projections = (self.q_proj(hidden_states), self.k_proj(hidden_states), self.v_proj(hidden_states))
            retention_raw = self.f_proj(hidden_states).view(B, T, H, K)
            omega_raw = self.omega_proj(hidden_states).view(B, T, H, K)
            r_raw = self.r_proj(hidden_states)
        convs = (self.q_conv1d, self.k_conv1d, self.v_conv1d)
        if stateful:
            tails, outs = [], []
            for i, (x, conv) in enumerate(zip(projections, convs)):
                xc, tail = conv_input_with_tail(x, state.conv[i] if state is not None else None)
                outs.append(conv(xc)[:, CONV_TAIL:].contiguous())
                tails.append(tail)
            q, k, v = outs
        else:
            q, k, v = (conv(x.contiguous()) for x, conv in zip(projections, convs))
        q, k, v = q.reshape(B, T, H, K), k.reshape(B, T, H, K), v.reshape(B, T, H, V)
        A_log = as_f32(self, "A_log", self.A_log)
        dt_bias = as_f32(self, "dt_bias", self.dt_bias).view(H, K)
        mu_param = as_f32(self, "mu_param", self.initial_precision_param)
        new_state = None
        scale = float(K ** -0.5)
        if not stateful:
            # normalisation -> frontend -> gain fused (the reference's three ops, same results)
            q_memory, k_memory, g_cumsum, kappa = diag_kdn_front(q, k, retention_raw, omega_raw, r_raw, A_log,
                                                                 dt_bias, mu_param)
            # the f32 recurrence is stored at the value dtype, as the reference's .to(v.dtype) does
            output = _chunk_kalman_as(q_memory, k_memory, kappa, v, g_cumsum, scale, out_dtype=v.dtype)
        else:
            if T == 1 and not torch.is_grad_enabled():  # gain and memory of one token in one launch
                q_memory, k_gain, k_memory = _diag_kdn_normalize(q, k)
                g_cumsum, alpha, omega, r, initial_precision = _diag_kdn_frontend_precumsum_paired(
                    retention_raw, omega_raw, r_raw, A_log, dt_bias, mu_param)
                prec0 = state.precision if state is not None else initial_precision
                inplace = state is not None and state.inplace
                if state is None:
                    memory = torch.zeros(B, H, K, V, device=q.device, dtype=torch.float32)
                else:
                    memory = state.memory if inplace else state.memory.clone()
                pin = prec0.float().view(1, H, 1).expand(B, H, K) if prec0.ndim == 1 else prec0
                output, precision = kdn_kalman_step(
                    q_memory, k_memory, v, g_cumsum, state=memory, precision=pin.contiguous(), alpha=alpha,
                    omega=omega, r=r, k_gain=k_gain, info_scale=float(K), scale=scale, out_dtype=v.dtype,
                    precision_out=state.precision_scratch() if inplace else None)
            else:
                q_memory, k_memory, g_cumsum, kappa, precision = diag_kdn_front(
                    q, k, retention_raw, omega_raw, r_raw, A_log, dt_bias, mu_param,
                    initial_precision=state.precision if state is not None else None, output_final_state=True)
                output, memory = _chunk_kalman_as(q_memory, k_memory, kappa, v, g_cumsum, scale,
                                                  initial_state=state.memory if state is not None else None,
                                                  output_final_state=True, out_dtype=v.dtype)
            new_state = carry_state(state, tails, memory, precision, T)
            if not use_cache:
                new_state = None
        if gate is None:
            gate = self.g_proj(hidden_states)
        output = self.o_norm(output, gate.view(B, T, H, V))
        return linear(output.reshape(B, T, self.value_dim), self.o_proj.weight), None, new_state


__all__ = ("DiagonalKalmanDeltaNetwork", "ShortConvolution")
