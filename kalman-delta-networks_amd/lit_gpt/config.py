"""Model configuration of the KDN block stack (``lit_gpt/config.py`` of the reference,
ngocbh/kalman-delta-networks, restricted to the KDN mixers).

Same field names, defaults and derived values (``padded_vocab_size``, ``n_query_groups``,
``head_size``, ``from_name``) as reference config.py:17-101; ``name_to_config`` holds the two KDN
configurations (reference config.py:136-183).  ``norm_class`` resolves to this package's
``FusedRMSNorm``; attention/GDN2 mixers are outside this build and are rejected by ``Block``.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Literal, Optional


def find_multiple(n: int, k: int) -> int:
    """Smallest multiple of k that is >= n (reference utils.py:26-30)."""
    assert k > 0
    return n if n % k == 0 else n + k - (n % k)


@dataclass
class Config:
    org: str = "Lightning-AI"
    name: str = "lit-GPT"
    block_size: int = 4096
    vocab_size: int = 50254
    padding_multiple: int = 64
    padded_vocab_size: Optional[int] = None
    n_layer: int = 16
    n_head: int = 32
    n_embd: int = 4096
    rotary_percentage: float = 0.25
    parallel_residual: bool = True
    bias: bool = True
    local_window: int = -1
    mlp: bool = True
    gdn2_per_layer: int = -1
    mixer_type: str = "gdn2"
    kdn_omega_min: float = 0.0
    kdn_r_min: float = 0.01
    kdn_info_scale: Optional[float] = None
    nope: bool = False
    mamba_init: bool = False
    n_query_groups: Optional[int] = None
    shared_attention_norm: bool = False
    _norm_class: Literal["LayerNorm", "RMSNorm", "FusedRMSNorm"] = "LayerNorm"
    norm_eps: float = 1e-5
    _mlp_class: Literal["LLaMAMLP"] = "LLaMAMLP"
    intermediate_size: Optional[int] = None
    condense_ratio: int = 1

    def __post_init__(self):
        assert self.n_embd % self.n_head == 0
        if self.padded_vocab_size is None:
            self.padded_vocab_size = find_multiple(self.vocab_size, self.padding_multiple)
        if self.n_query_groups is not None:
            assert self.n_head % self.n_query_groups == 0
        else:
            self.n_query_groups = self.n_head
        if self.intermediate_size is None:
            if self._mlp_class == "LLaMAMLP":
                raise ValueError("The config needs to set the `intermediate_size`")
            self.intermediate_size = 4 * self.n_embd

    @property
    def head_size(self) -> int:
        return self.n_embd // self.n_head

    @classmethod
    def from_name(cls, name: str, **kwargs: Any) -> "Config":
        conf_dict = name_to_config[name].copy()
        conf_dict.update(kwargs)
        return cls(**conf_dict)

    @property
    def mlp_class(self):
        from . import model
        return getattr(model, self._mlp_class)

    @property
    def norm_class(self):
        if self._norm_class in ("RMSNorm", "FusedRMSNorm"):
            from .rmsnorm import FusedRMSNorm
            return FusedRMSNorm
        import torch
        return getattr(torch.nn, self._norm_class)


def _kdn_config(name: str, mixer_type: str, intermediate_size: int) -> dict:
    return dict(org="yale", name=name, block_size=4096, vocab_size=32000, padding_multiple=64, gdn2_per_layer=1,
                mixer_type=mixer_type, kdn_omega_min=0.0, kdn_r_min=0.01, kdn_info_scale=128.0, n_layer=18,
                n_head=18, n_embd=2304, rotary_percentage=1.0, parallel_residual=False, bias=False,
                _norm_class="FusedRMSNorm", norm_eps=1e-5, _mlp_class="LLaMAMLP",
                intermediate_size=intermediate_size, local_window=2048, mamba_init=True)


configs = [
    # iso: 1,449,848,592 parameters in total, transformer.h 1,302,390,288
    _kdn_config("iso_kdn_1.3B", "iso_kdn", 7208),
    # diag: 1,449,806,796 parameters in total, transformer.h 1,302,348,492
    _kdn_config("diag_kdn_1.3B", "diag_kdn", 7128),
]

name_to_config = {config["name"]: config for config in configs}

__all__ = ("Config", "configs", "name_to_config", "find_multiple")
