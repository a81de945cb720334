"""Helpers shared by the GPU parity tests (inputs, oracle calls, error metric)."""
from __future__ import annotations

import math
import sys

import pytest
import torch

LN2 = math.log(2.0)


def gpu_or_skip():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    return torch.device("cuda:0")


def rel(x, ref) -> float:
    """max|x - ref| / max|ref| (the parity metric of the north star).

    When the reference is identically zero (e.g. the gate gradient of a single token,
    whose state does not depend on its own retention) the absolute error is returned."""
    x = x.detach().double().cpu()
    ref = ref.detach().double().cpu()
    scale = float(ref.abs().max())
    if scale == 0.0:
        return float((x - ref).abs().max())
    return float((x - ref).abs().max()) / scale


def log(msg: str):
    print(msg, flush=True)
    sys.stdout.flush()


def chunk_prefix_base2(ell: torch.Tensor, chunk: int) -> torch.Tensor:
    """Chunk-local inclusive prefix of a natural-log gate [B,T,H,K], in base 2."""
    T = ell.shape[1]
    parts = [ell[:, c:c + chunk].cumsum(1) for c in range(0, T, chunk)]
    return torch.cat(parts, 1) / LN2


def reverse_chunk_sum(dg: torch.Tensor, chunk: int) -> torch.Tensor:
    """Reverse (suffix) sum within chunks: maps a prefix cotangent to a per-token one."""
    T = dg.shape[1]
    parts = [dg[:, c:c + chunk].flip(1).cumsum(1).flip(1) for c in range(0, T, chunk)]
    return torch.cat(parts, 1)


def memory_inputs(seed, B, T, H, K, V, *, diag: bool, ell_mean=-0.13, ell_std=0.05):
    """Memory-scan inputs exactly representable at the HIP boundary: q, k unit-norm then
    rounded to bf16; v bf16; kappa (diag) or beta (iso) fp32; per-token log-gate ell fp32."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=g)
    k = torch.randn(B, T, H, K, generator=g)
    q = (q / q.norm(dim=-1, keepdim=True)).bfloat16()
    k = (k / k.norm(dim=-1, keepdim=True)).bfloat16()
    v = torch.randn(B, T, H, V, generator=g).bfloat16()
    ell = (ell_mean + ell_std * torch.randn(B, T, H, K, generator=g)).clamp(max=0.0)
    if diag:
        kap = 0.5 * torch.rand(B, T, H, K, generator=g) * k.float()
    else:
        kap = 0.2 + 0.8 * torch.rand(B, T, H, generator=g)
    do = torch.randn(B, T, H, V, generator=g)
    return q, k, v, ell, kap, do
