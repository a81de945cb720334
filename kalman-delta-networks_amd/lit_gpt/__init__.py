"""MI355X-native drop-in for the Kalman Delta Network scan path of lit_gpt (kdn_ops).

The package root exports what the reference's lit_gpt/__init__.py:1-3 does for this path
(``pretrain.py:37`` imports ``FusedCrossEntropyLoss`` from here); the tokenizer is not part of it.
"""
from .config import Config
from .fused_cross_entropy import FusedCrossEntropyLoss
from .model import GPT

__all__ = ["GPT", "Config", "FusedCrossEntropyLoss"]
