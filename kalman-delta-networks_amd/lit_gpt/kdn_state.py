"""Recurrent state of a KDN layer, for chunked long-context prefill and token-by-token decode.

The reference runs its KDN layers on fixed-length sequences only (``model.py:104,184`` refuse
caching; ``iso_kdn.py:221-257`` and ``diag_kdn.py:247-283`` reject ``past_key_values`` and
``use_cache``).  A KDN layer is a recurrence, so its whole history is a fixed-size state:

* ``conv``: the inputs of the width-4 causal short convolutions for the last 3 tokens, one
  [B, 3, C] tensor per convolution (isotropic: the packed q|k|v projection, C = 3D; diagonal:
  the q, k and v projections, C = D each), zeros before the first token (the convolution's own
  zero padding);
* ``memory``: the associative memory S [B,H,K,V] fp32 (the chunked scan's initial / final
  state; zeros before the first token);
* ``precision``: the Kalman precision 1/p after the last token, [B,H] (isotropic) or [B,H,K]
  (diagonal) fp32; before the first token it is the layer's learned initial precision.

A sequence split into segments, each run from the previous segment's state, gives the outputs
of the whole sequence run at once (up to rounding order), and gradients flow through the state
when the segments are differentiated together.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch

CONV_TAIL = 3  # width-4 short convolution: 3 earlier inputs


@dataclass
class KDNLayerState:
    """``inplace=True`` makes a layer advance this object's own buffers (inference only), so their
    addresses stay fixed across calls, as a replayed HIP graph needs; otherwise every call
    returns a new state and leaves this one unchanged."""
    conv: tuple
    memory: torch.Tensor
    precision: torch.Tensor
    seen_tokens: int = 0
    inplace: bool = False
    _scratch: Optional[torch.Tensor] = field(default=None, repr=False)

    def detach(self) -> "KDNLayerState":
        """The same state cut from the autograd graph (truncated back-propagation)."""
        return KDNLayerState(tuple(c.detach() for c in self.conv), self.memory.detach(), self.precision.detach(),
                             self.seen_tokens)

    def precision_scratch(self) -> torch.Tensor:
        """A second precision buffer for a kernel that must not read and write the same one."""
        if self._scratch is None:
            self._scratch = torch.empty_like(self.precision)
        return self._scratch


def carry_state(state, conv, memory, precision, T: int):
    """The state after T more tokens: a new KDNLayerState, or ``state`` itself advanced in place
    (its buffers overwritten) when it is an in-place state."""
    if state is not None and state.inplace:
        if torch.is_grad_enabled():
            raise RuntimeError("in-place KDN layer states are for inference; run under torch.no_grad()")
        for c, n in zip(state.conv, conv):
            if n is not c:  # a single-token step may already have advanced the buffer itself
                c.copy_(n)
        if memory is not state.memory:
            state.memory.copy_(memory)
        if precision is not state.precision:
            state.precision.copy_(precision)
        state.seen_tokens += T
        return state
    return KDNLayerState(tuple(conv), memory, precision, (state.seen_tokens if state is not None else 0) + T)


def conv_input_with_tail(x: torch.Tensor, tail):
    """[tail, x] along time and the new tail (the last 3 inputs).  ``tail`` None means zeros:
    the convolution of the concatenation, with its first 3 outputs dropped, is the convolution
    of x continued from the earlier inputs."""
    B, T, C = x.shape
    if tail is None:
        tail = x.new_zeros(B, CONV_TAIL, C)
    elif tail.shape != (B, CONV_TAIL, C):
        raise ValueError(f"convolution state must have shape {(B, CONV_TAIL, C)}, got {tuple(tail.shape)}")
    xc = torch.cat([tail.to(x.dtype), x], dim=1)
    return xc, xc[:, -CONV_TAIL:]


def check_state(state, B: int, H: int, K: int, V: int, n_conv: int, precision_shape, device) -> None:
    if not isinstance(state, KDNLayerState):
        raise TypeError(f"past_key_values must be a KDNLayerState, got {type(state).__name__}")
    if len(state.conv) != n_conv:
        raise ValueError(f"expected {n_conv} convolution states, got {len(state.conv)}")
    if state.memory.shape != (B, H, K, V) or state.memory.dtype != torch.float32:
        raise ValueError(f"memory state must be fp32 [{B},{H},{K},{V}], got {state.memory.dtype} "
                         f"{tuple(state.memory.shape)}")
    if state.precision.shape != tuple(precision_shape) or state.precision.dtype != torch.float32:
        raise ValueError(f"precision state must be fp32 {tuple(precision_shape)}, got {state.precision.dtype} "
                         f"{tuple(state.precision.shape)}")
    for t in (*state.conv, state.memory, state.precision):
        if t.device != device:
            raise ValueError("the layer state must live on the hidden states' device")


__all__ = ("KDNLayerState", "carry_state", "conv_input_with_tail", "check_state", "CONV_TAIL")
