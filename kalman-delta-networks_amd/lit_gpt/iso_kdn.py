"""Isotropic KDN mixer layer on MI355X (``IsotropicKalmanDeltaNetwork``).

Mirrors ``lit_gpt/iso_kdn.py`` of the reference (ngocbh/kalman-delta-networks): the same
constructor arguments and checks (:87-156), the same parameter names and shapes after the
reference's projection packing (``qkv_pack.projection_weight`` [3D, hidden],
``qkv_pack.convolution_weight`` [3D, 4], ``f_omega_r_proj.weight`` [d + 2H, hidden],
``f_proj.1``, ``omega_proj.bias``, ``r_proj.bias``, ``A_log``, ``dt_bias``, ``g_proj``,
``o_norm.weight``, ``o_proj``, ``initial_precision_param``), so a reference state dict loads,
and the same forward composition (:262-314): packed q|k|v projection -> SiLU short convolution
-> gate frontend -> scalar Kalman gain -> chunked memory scan -> sigmoid-gated RMS norm ->
output projection.  Projections are torch GEMMs; everything else runs in ``libkdn_hip.so``.
The reference's RNG-order-preserving construction is not reproduced (random init differs).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import nn

from ._inference import as_f32, linear, packed_weight, use_packed
from .kdn_ops.gated_norm import FusedRMSNormGated
from .kdn_ops.iso_kdn_chunk import _chunk_kda_precumsum_paired, _iso_kdn_gate_precumsum_paired, iso_kdn_front
from .kdn_ops.short_conv import qkv_causal_conv1d, short_conv_step
from .kdn_ops.step import kdn_kalman_step
from .kdn_state import CONV_TAIL, carry_state, check_state, conv_input_with_tail

_SUPPORTED_HEAD_DIMS = (64, 128)
_INITIAL_PRECISION = 1.0
_INITIAL_PRECISION_FLOOR = 0.1


def validate_training_dtype(variant: str, *, training: bool, hidden_dtype: torch.dtype) -> None:
    """Training runs under CUDA bf16 autocast on fp32/bf16 hidden states (reference iso_kdn.py:51-62)."""
    if not training:
        return
    if not torch.is_autocast_enabled("cuda") or torch.get_autocast_dtype("cuda") != torch.bfloat16:
        raise TypeError(f"{variant} KDN training requires CUDA BF16 autocast")
    if hidden_dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"{variant} KDN training requires FP32 or BF16 hidden states under CUDA BF16 autocast")


def initial_precision_inverse() -> float:
    """softplus^-1(P0 - floor): the raw value that gives the initial precision 1.0."""
    return math.log(math.expm1(_INITIAL_PRECISION - _INITIAL_PRECISION_FLOOR))


def decay_parameters(num_heads: int, gate_dim: int):
    """A_log ~ log U(1, 16) per head; dt_bias = softplus^-1(dt), dt log-uniform in [1e-3, 0.1]
    (reference iso_kdn.py:173-185)."""
    A_log = nn.Parameter(torch.log(torch.empty(num_heads, dtype=torch.float32).uniform_(1, 16)))
    dt = torch.exp(torch.rand(gate_dim, dtype=torch.float32) * (math.log(0.1) - math.log(0.001))
                   + math.log(0.001)).clamp(min=1e-4)
    dt_bias = nn.Parameter(dt + torch.log(-torch.expm1(-dt)))
    A_log._no_weight_decay = True
    dt_bias._no_weight_decay = True
    return A_log, dt_bias


class PackedQKV(nn.Module):
    """Canonical q|k|v projection and depthwise-convolution weights (reference iso_kdn_chunk.py:573-660)."""

    def __init__(self, hidden_size: int, device=None, dtype=None):
        super().__init__()
        self.hidden_size = int(hidden_size)
        self.out_features = 3 * self.hidden_size
        self.kernel_size = 4
        self.projection_weight = nn.Parameter(torch.empty(self.out_features, self.hidden_size, device=device,
                                                          dtype=dtype))
        self.convolution_weight = nn.Parameter(torch.empty(self.out_features, 4, device=device, dtype=dtype))

    def forward(self, x):
        return qkv_causal_conv1d(F.linear(x, self.projection_weight), self.convolution_weight)


class PackedLinear(nn.Module):
    """One biasless weight split into output segments (reference iso_kdn_chunk.py:481-534)."""

    def __init__(self, in_features: int, segment_sizes, device=None, dtype=None):
        super().__init__()
        self.in_features = int(in_features)
        self.segment_sizes = tuple(int(s) for s in segment_sizes)
        self.out_features = sum(self.segment_sizes)
        self.weight = nn.Parameter(torch.empty(self.out_features, self.in_features, device=device, dtype=dtype))

    def forward_packed(self, x):
        return F.linear(x, self.weight)


class _Bias(nn.Module):
    """Holds only a bias (the reference's packed-slice modules own no weight)."""

    def __init__(self, n: int, device=None, dtype=None):
        super().__init__()
        self.bias = nn.Parameter(torch.zeros(n, device=device, dtype=dtype))


class IsotropicKalmanDeltaNetwork(nn.Module):
    """Isotropic KDN mixer (reference iso_kdn.py:84-314), plus an optional carried state."""

    def __init__(self, hidden_size: int = 2304, head_dim: int = 128, num_heads: int = 18, expand_v: float = 1.0,
                 num_v_heads=None, use_short_conv: bool = True, conv_size: int = 4, conv_bias: bool = False,
                 omega_min: float = 0.0, r_min: float = 0.01, info_scale=None, norm_eps: float = 1e-5,
                 layer_idx=None):
        if head_dim not in _SUPPORTED_HEAD_DIMS:
            raise ValueError(f"unsupported Isotropic KDN head_dim {head_dim}; expected one of {_SUPPORTED_HEAD_DIMS}")
        if hidden_size != head_dim * num_heads:
            raise ValueError("Isotropic KDN hidden_size must equal head_dim * num_heads; "
                             f"got hidden_size={hidden_size}, head_dim={head_dim}, num_heads={num_heads}")
        if (num_heads if num_v_heads is None else num_v_heads) != num_heads:
            raise ValueError("num_v_heads must equal num_heads for Isotropic KDN")
        if float(expand_v) != 1.0:
            raise ValueError(f"expand_v must be 1.0 for Isotropic KDN, got {expand_v!r}")
        if not use_short_conv or conv_size != 4 or conv_bias:
            raise ValueError("Isotropic KDN requires the biasless width-4 short-convolution path")
        if not (omega_min >= 0 and math.isfinite(omega_min)):
            raise ValueError(f"omega_min must be nonnegative and finite, got {omega_min!r}")
        if not (r_min > 0 and math.isfinite(r_min)):
            raise ValueError(f"r_min must be positive and finite, got {r_min!r}")
        super().__init__()
        self.omega_min = float(omega_min)
        self.r_min = float(r_min)
        self.info_scale = float(head_dim) if info_scale is None else float(info_scale)
        self.hidden_size = hidden_size
        self.head_dim = self.head_k_dim = self.head_v_dim = head_dim
        self.num_heads = self.num_v_heads = num_heads
        self.key_dim = self.value_dim = self.gate_dim = num_heads * head_dim
        self.layer_idx = layer_idx

        self.qkv_pack = PackedQKV(hidden_size)
        self.f_omega_r_proj = PackedLinear(hidden_size, (head_dim, num_heads, num_heads))
        self.f_proj = nn.Sequential(nn.Identity(), nn.Linear(head_dim, self.gate_dim, bias=False))
        self.omega_proj = _Bias(num_heads)
        self.r_proj = _Bias(num_heads)
        self.A_log, self.dt_bias = decay_parameters(num_heads, self.gate_dim)
        self.g_proj = nn.Sequential(nn.Linear(hidden_size, head_dim, bias=False),
                                    nn.Linear(head_dim, self.value_dim, bias=True))
        self.o_norm = FusedRMSNormGated(head_dim, activation="sigmoid", eps=norm_eps)
        self.o_proj = nn.Linear(self.value_dim, hidden_size, bias=False)
        self.initial_precision_param = nn.Parameter(torch.full((num_heads,), initial_precision_inverse(),
                                                               dtype=torch.float32))
        self.initial_precision_param._no_weight_decay = True
        self.reset_parameters()

    @torch.no_grad()
    def reset_parameters(self):
        """Random init of the packed weights (Linear-style uniform; conv like nn.Conv1d depthwise)."""
        for wgt in (self.qkv_pack.projection_weight, self.f_omega_r_proj.weight):
            nn.init.kaiming_uniform_(wgt, a=math.sqrt(5))
        nn.init.kaiming_uniform_(self.qkv_pack.convolution_weight, a=math.sqrt(5))
        bound = 1.0 / math.sqrt(self.hidden_size)
        self.omega_proj.bias.uniform_(-bound, bound)
        self.r_proj.bias.uniform_(-bound, bound)

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
            raise ValueError("IsotropicKalmanDeltaNetwork supports only fixed-length sequences (with an optional "
                             f"carried state); unsupported arguments: {requested}")
        if hidden_states.ndim != 3 or hidden_states.shape[-1] != self.hidden_size:
            raise ValueError(f"hidden_states must have shape [B,T,{self.hidden_size}], "
                             f"got {tuple(hidden_states.shape)}")
        if hidden_states.shape[0] == 0 or hidden_states.shape[1] == 0:
            raise ValueError("Isotropic KDN requires non-empty batch and sequence dimensions")
        if torch.is_grad_enabled() and hidden_states.shape[1] < 2:
            raise ValueError("differentiable Isotropic KDN training requires sequence length >= 2; "
                             "the exact one-token convolution update is inference-only")
        if not hidden_states.is_cuda:
            raise ValueError("IsotropicKalmanDeltaNetwork requires CUDA hidden_states")
        validate_training_dtype("Isotropic", training=self.training, hidden_dtype=hidden_states.dtype)
        B, T, _ = hidden_states.shape
        H, K = self.num_heads, self.head_k_dim
        stateful = past_key_values is not None or bool(use_cache)
        state = past_key_values
        if state is not None:
            check_state(state, B, H, K, self.head_v_dim, 1, (B, H), hidden_states.device)
        gate = None
        if use_packed(hidden_states, self):  # a few rows without autograd: the three input GEMMs as one
            # rows padded to a multiple of 8, so each token's q|k|v slice starts 16-byte aligned (the
            # single-token convolution kernel's vector loads)
            w_in = packed_weight(self, "in_proj", (self.qkv_pack.projection_weight, self.f_omega_r_proj.weight,
                                                   self.g_proj[0].weight), row_multiple=8)
            sizes = (self.qkv_pack.out_features, self.head_v_dim + 2 * H, self.head_v_dim)
            x_lin, packed, g_hidden = linear(hidden_states, w_in).split(sizes + (w_in.shape[0] - sum(sizes),),
                                                                         dim=-1)[:3]
            gate = linear(g_hidden, self.g_proj[1].weight, self.g_proj[1].bias)
        else:
            x_lin = F.linear(hidden_states, self.qkv_pack.projection_weight)
            packed = self.f_omega_r_proj.forward_packed(hidden_states)
        cw = self.qkv_pack.convolution_weight
        if (stateful and T == 1 and state is not None and state.inplace and not torch.is_grad_enabled()
                and state.conv[0].dtype == x_lin.dtype and x_lin.data_ptr() % 16 == 0
                and (B == 1 or x_lin.stride(0) % 8 == 0)
                and x_lin.stride(-1) == 1 and cw.is_contiguous()):
            # decode step: one launch convolves the token with the carried inputs and advances them
            y = short_conv_step(x_lin, state.conv[0], cw)
            d = y.shape[-1] // 3
            q, k, v = y[..., :d], y[..., d:2 * d], y[..., 2 * d:]
            conv_tail = state.conv[0]
        elif stateful:
            x_proj, conv_tail = conv_input_with_tail(x_lin, state.conv[0] if state is not None else None)
            q, k, v = (t[:, CONV_TAIL:] for t in qkv_causal_conv1d(x_proj, cw))
        else:
            q, k, v = qkv_causal_conv1d(x_lin.contiguous(), self.qkv_pack.convolution_weight)
        f_hidden, omega_r_raw = packed.split((self.head_v_dim, 2 * H), dim=-1)
        g_raw = linear(f_hidden, self.f_proj[1].weight)
        q, k = q.reshape(B, T, H, K), k.reshape(B, T, H, K)
        v = v.reshape(B, T, H, self.head_v_dim)
        g_raw = g_raw.view(B, T, H, K)
        gate_args = (g_raw, omega_r_raw, as_f32(self, "omega_bias", self.omega_proj.bias),
                     as_f32(self, "r_bias", self.r_proj.bias), as_f32(self, "A_log", self.A_log),
                     as_f32(self, "dt_bias", self.dt_bias), as_f32(self, "mu_param", self.initial_precision_param),
                     self.omega_min, self.r_min)
        new_state = None
        if not stateful:  # gate -> gain fused (the reference's two ops, same results)
            g_cumsum, gain = iso_kdn_front(*gate_args, head_dim=K, info_scale=self.info_scale)
            output = _chunk_kda_precumsum_paired(q=q, k=k, v=v, g_cumsum=g_cumsum, beta=gain)
        else:
            if T == 1 and not torch.is_grad_enabled():  # gain and memory of one token in one launch
                g_cumsum, a, omega, r, initial_precision = _iso_kdn_gate_precumsum_paired(*gate_args)
                prec0 = state.precision if state is not None else initial_precision
                inplace = state is not None and state.inplace
                if state is None:
                    memory = torch.zeros(B, H, K, self.head_v_dim, device=q.device, dtype=torch.float32)
                else:
                    memory = state.memory if inplace else state.memory.clone()
                output, precision = kdn_kalman_step(
                    q, k, v, g_cumsum, state=memory, precision=prec0.float().expand(B, H).contiguous(), a=a,
                    omega=omega, r=r, info_scale=self.info_scale,
                    precision_out=state.precision_scratch() if inplace else None)
            else:
                g_cumsum, gain, precision = iso_kdn_front(
                    *gate_args, head_dim=K, info_scale=self.info_scale,
                    initial_precision=state.precision if state is not None else None, output_final_state=True)
                output, memory = _chunk_kda_precumsum_paired(
                    q=q, k=k, v=v, g_cumsum=g_cumsum, beta=gain,
                    initial_state=state.memory if state is not None else None, output_final_state=True)
            new_state = carry_state(state, (conv_tail,), memory, precision, T)
            if not use_cache:
                new_state = None
        if gate is None:
            gate = self.g_proj(hidden_states)
        output = self.o_norm(output, gate.view(B, T, H, self.head_v_dim))
        return linear(output.reshape(B, T, self.value_dim), self.o_proj.weight), None, new_state


__all__ = ("IsotropicKalmanDeltaNetwork", "PackedQKV", "PackedLinear")
