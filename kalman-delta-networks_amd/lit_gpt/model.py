"""The KDN block stack (``GPT`` / ``Block`` / ``LLaMAMLP`` / ``SwiGLU``) on MI355X.

Mirrors ``lit_gpt/model.py`` of the reference (ngocbh/kalman-delta-networks) for the configurations
whose every layer is a KDN mixer (``gdn2_per_layer=1``, ``mixer_type`` "iso_kdn" / "diag_kdn"):

* ``GPT`` (model.py:27-165): ``wte`` -> blocks -> ``ln_f`` -> ``lm_head``, same module names, so
  a reference state dict loads; KV caching is rejected for KDN mixers as in the reference.  The
  rotary cache the reference builds is not consumed by KDN blocks and is not built here.
  Beyond the reference, the layers' recurrent state can be carried between calls (``state=`` /
  ``return_state=True``) for segmented prefill and token-by-token decoding.
* ``Block`` (model.py:217-298): pre-norm residual ``x + mixer(norm_1(x))`` then
  ``x + mlp(norm_2(x))`` (``parallel_residual=False``).
* ``LLaMAMLP`` / ``SwiGLU`` (model.py:415-464): w3(silu(w1 x) * w2 x).
* ``GPT._init_weights`` (model.py:47-85): the mamba / GPT-NeoX initialisation.

Norms run in ``libkdn_hip.so`` (``FusedRMSNorm``); the mixers are this package's KDN layers;
the dense projections are torch GEMMs (hipBLASLt).
"""
from __future__ import annotations

import math
from typing import Any, Optional

import torch
import torch.nn.functional as F
from torch import nn

from ._inference import linear, packed_weight, swiglu_gate, use_packed
from .config import Config


class GPT(nn.Module):
    def __init__(self, config: Config) -> None:
        super().__init__()
        assert config.padded_vocab_size is not None
        self.config = config
        self.lm_head = nn.Linear(config.n_embd, config.padded_vocab_size, bias=False)
        self.transformer = nn.ModuleDict(dict(
            wte=nn.Embedding(config.padded_vocab_size, config.n_embd),
            h=nn.ModuleList(Block(config, i) for i in range(config.n_layer)),
            ln_f=config.norm_class(config.n_embd, eps=config.norm_eps),
        ))
        self.max_len = config.block_size
        self.mamba_init = config.mamba_init

    def _init_weights(self, module: nn.Module, n_layer) -> None:
        """Meant to be used with ``gpt.apply(partial(gpt._init_weights, n_layer=...))``."""
        if isinstance(module, nn.Embedding):
            if self.mamba_init:
                nn.init.normal_(module.weight, std=0.02)
            else:
                nn.init.normal_(module.weight, mean=0.0, std=math.sqrt(2.0 / 5 / self.config.n_embd))
        elif isinstance(module, nn.Linear):
            if self.mamba_init:
                if module.bias is not None and not getattr(module.bias, "_no_reinit", False):
                    nn.init.zeros_(module.bias)
            else:
                nn.init.normal_(module.weight, mean=0.0, std=math.sqrt(2.0 / 5 / self.config.n_embd))
                if module.bias is not None:
                    nn.init.zeros_(module.bias)
        for name, p in module.named_parameters():
            if (name in ("out_proj.weight", "fc2.weight") or (name == "proj.weight" and isinstance(module, LLaMAMLP))
                    or (name == "w3.weight" and isinstance(module, SwiGLU))):
                if self.mamba_init:
                    n_residuals_per_layer = 1 if not self.config.mlp else 2
                    nn.init.kaiming_uniform_(p, a=math.sqrt(5))
                    with torch.no_grad():
                        p /= math.sqrt(n_residuals_per_layer * n_layer)
                else:
                    nn.init.normal_(p, mean=0.0, std=1 / math.sqrt(self.config.n_embd) / n_layer)
        # the diagonal layer starts from isotropic process noise
        if getattr(module, "_kdn_omega_zero", False):
            nn.init.zeros_(module.weight)
            if module.bias is not None:
                nn.init.zeros_(module.bias)

    def init_weights(self) -> None:
        """Apply ``_init_weights`` to every module, as the reference's training script does."""
        self.apply(lambda m: self._init_weights(m, self.config.n_layer))

    def reset_cache(self) -> None:
        self.max_len = self.config.block_size

    def forward(self, idx: torch.Tensor, max_seq_length: Optional[int] = None,
                input_pos: Optional[torch.Tensor] = None, *, state: Optional[list] = None,
                return_state: bool = False):
        """Logits [B,T,vocab].  KV caching by position (``input_pos``) is refused as in the reference.

        State carry (not in the reference): ``state`` is the list of per-layer ``KDNLayerState``
        after the earlier tokens of these sequences (from a previous call with
        ``return_state=True``), and ``return_state=True`` returns ``(logits, new_state)``.  Feeding
        a sequence in segments, or one token at a time under ``torch.no_grad()``, gives the logits
        of the whole sequence."""
        if input_pos is not None:
            raise ValueError("KDN mixers do not support KV caching (carry the recurrent state with "
                             "state= / return_state=True instead)")
        if max_seq_length is None:
            max_seq_length = self.config.block_size
        if state is not None and len(state) != len(self.transformer.h):
            raise ValueError(f"state must hold one entry per layer ({len(self.transformer.h)}), got {len(state)}")
        stateful = return_state or state is not None
        states = list(state) if state is not None else [None] * len(self.transformer.h)
        x = self.transformer.wte(idx)
        for i, block in enumerate(self.transformer.h):
            x, new = block(x, None, max_seq_length, kv_cache=states[i], use_state=stateful)
            states[i] = new
        x = self.transformer.ln_f(x)
        logits = linear(x, self.lm_head.weight)
        return (logits, states) if return_state else logits

    @classmethod
    def from_name(cls, name: str, **kwargs: Any) -> "GPT":
        return cls(Config.from_name(name, **kwargs))


class Block(nn.Module):
    def __init__(self, config: Config, layer_idx: int) -> None:
        super().__init__()
        self.norm_1 = config.norm_class(config.n_embd, eps=config.norm_eps)
        self.use_gdn2 = layer_idx % config.gdn2_per_layer == 0 if config.gdn2_per_layer > 0 else False
        self.is_iso_kdn = self.use_gdn2 and config.mixer_type == "iso_kdn"
        self.is_diag_kdn = self.use_gdn2 and config.mixer_type == "diag_kdn"
        kwargs = dict(hidden_size=config.n_embd, head_dim=config.head_size, num_heads=config.n_head, expand_v=1.0,
                      omega_min=config.kdn_omega_min, r_min=config.kdn_r_min, info_scale=config.kdn_info_scale,
                      norm_eps=config.norm_eps, layer_idx=layer_idx)
        if self.is_iso_kdn:
            from .iso_kdn import IsotropicKalmanDeltaNetwork
            self.attn = IsotropicKalmanDeltaNetwork(**kwargs)
        elif self.is_diag_kdn:
            from .diag_kdn import DiagonalKalmanDeltaNetwork
            self.attn = DiagonalKalmanDeltaNetwork(**kwargs)
        else:
            raise ValueError("only KDN mixer layers are built here "
                             f"(mixer_type={config.mixer_type!r}, gdn2_per_layer={config.gdn2_per_layer})")
        if not config.shared_attention_norm and config.mlp and not config.parallel_residual:
            self.norm_2 = config.norm_class(config.n_embd, eps=config.norm_eps)
        if config.mlp:
            self.mlp = config.mlp_class(config)
        self.config = config

    def forward(self, x, rope=None, max_seq_length=None, mask=None, input_pos=None, kv_cache=None, *,
                use_state=False):
        """``kv_cache`` carries the mixer's ``KDNLayerState``; with ``use_state`` the second output is
        the state after these tokens (None otherwise)."""
        if input_pos is not None:
            raise ValueError("KDN mixers do not support KV caching")
        n_1 = self.norm_1(x)
        h, _, new_kv_cache = self.attn(n_1, attention_mask=mask, past_key_values=kv_cache, use_cache=use_state)
        if self.config.parallel_residual:
            assert self.config.shared_attention_norm
            if self.config.mlp:
                h = h + self.mlp(n_1)
            x = x + h
        else:
            x = x + h
            if self.config.mlp:
                x = x + self.mlp(self.norm_2(x))
        return x, new_kv_cache


class LLaMAMLP(nn.Module):
    def __init__(self, config: Config) -> None:
        super().__init__()
        self.swiglu = SwiGLU(config.n_embd, config.intermediate_size, bias=config.bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.swiglu(x)


class SwiGLU(nn.Module):
    def __init__(self, in_features, hidden_features, bias=False):
        super().__init__()
        self.w1 = nn.Linear(in_features, hidden_features, bias=bias)
        self.w2 = nn.Linear(in_features, hidden_features, bias=bias)
        self.w3 = nn.Linear(hidden_features, in_features, bias=bias)

    def forward(self, x):
        if self.w1.bias is None and self.w2.bias is None and use_packed(x, self):  # decode: w1 | w2 as one GEMM
            h = swiglu_gate(x, packed_weight(self, "w12", (self.w1.weight, self.w2.weight)))
            return linear(h, self.w3.weight, self.w3.bias)
        return self.w3(F.silu(self.w1(x)) * self.w2(x))


__all__ = ("GPT", "Block", "LLaMAMLP", "SwiGLU", "Config")
