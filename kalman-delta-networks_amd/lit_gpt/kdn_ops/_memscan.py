"""Stage-by-stage launch of the chunked memory scan (kdn_mem_fwd / kdn_mem_bwd).

Each stage is one kernel; launching them separately lets KernelTimer attribute time to
kernels.  Shared by the iso (kappa = beta k) and diag (explicit kappa) operators.
"""
from __future__ import annotations

import os

import torch

from . import _lib

# bits 1 | 2 in one call: the state pass with the readout fused (with chunk groups, fused into the
# groups that start from their true state; the first group's readout follows in the same call)
FWD_STAGES = ((1, "mem_intra_fwd"), (6, "mem_state_readout_fwd"))
# bits 0 | 1 | 2 in one call: with one chunk group the sequence runs in two chunk ranges, the second
# range's intra-chunk build on a second stream beside the first range's state pass (same results)
FWD_STAGES_OVERLAP = ((7, "mem_fwd_overlap"),)
NO_BACKWARD = 8  # stage bit: no backward follows, intermediates only the backward reads are not written


def state_groups(B: int, T: int, H: int, K: int, V: int) -> int:
    """Chunk groups of the serial state passes at this shape (1: one pass, readout fused)."""
    return int(_lib.load().kdn_mem_state_groups(B, T, H, K, V))
# bit 2: the chunk-parallel backward of every chunk (products with h and dh; solves and gradients of
# the chunks the forward factored); bits 4 | 8: the exact path's solves and gradients (flagged chunks)
BWD_STAGES = ((1, "mem_state_bwd"), (2, "mem_bwd_chunk"), (12, "mem_bwd_exact"))
# bits 1 | 2 in one call: with one chunk group the reverse pass runs in segments and each finished
# segment's chunk backward overlaps the next segment's pass on a second stream (same results)
BWD_STAGES_OVERLAP = ((3, "mem_state_chunk_bwd"), (12, "mem_bwd_exact"))
# the default of mem_bwd's ``overlap`` outside a KernelTimer (a profiler that averages per-kernel
# durations wants every kernel in its own call)
DEFAULT_OVERLAP = True


# What a training forward keeps for its backward; both give bit-identical gradients.
#  "save"       the intra-chunk WY factors, A^T and the per-chunk states h, delta (kdn_mem_saved_size
#               bytes, ~4.1 KB per token-head at K = V = 128: 1.21 GB at B4 T4096 H18), so the backward
#               starts at its own passes;
#  "recompute"  only the op's inputs (and the in-op norm's rstd), as the reference's autograd functions
#               keep them (iso_kdn_chunk.py:2206, diag_kdn_chunk.py:3253); the backward first rebuilds
#               the intermediates per chunk (the intra-chunk build, then the forward state pass without
#               its readout) before its own passes, as the reference re-runs recompute_w_u_fwd and the
#               state forward (iso_kdn_chunk.py:2101-2140, diag_kdn_chunk.py:3271-3277).
# The environment variable KDN_MEMORY_BACKWARD sets the mode a process starts with.
BACKWARD_MODES = ("save", "recompute")
_backward_mode = os.environ.get("KDN_MEMORY_BACKWARD", "save")
if _backward_mode not in BACKWARD_MODES:
    raise ValueError(f"KDN_MEMORY_BACKWARD must be one of {BACKWARD_MODES}, got {_backward_mode!r}")


def set_backward_mode(mode: str) -> str:
    """Select what the memory scan's forward keeps for the backward; returns the previous mode."""
    global _backward_mode
    if mode not in BACKWARD_MODES:
        raise ValueError(f"backward mode must be one of {BACKWARD_MODES}, got {mode!r}")
    prev, _backward_mode = _backward_mode, mode
    return prev


def backward_mode() -> str:
    return _backward_mode


def mem_fwd(q, k, kappa_or_beta, iso: bool, v, g_cumsum, scale: float, *, initial_state=None,
            output_final_state=False, out_dtype=torch.float32, need_backward=True, q_rstd=None, k_rstd=None,
            overlap=None):
    """q, k, v bf16 [B,T,H,*]; kappa [B,T,H,K] f32 (diag) or beta [B,T,H] f32 (iso).
    Returns (o, saved, final_state or None); with ``need_backward=False`` saved is not usable by
    mem_bwd (the intermediates only the backward reads are skipped).

    With ``q_rstd`` / ``k_rstd`` (f32 [B,T,H] outputs, the in-op L2 norm) q and k are the raw inputs:
    the scan normalises their rows as kdn_l2norm_fwd would and writes the rows' rstd for mem_bwd.

    ``overlap`` (default: unless a KernelTimer is timing each kernel) launches the intra-chunk build and
    the state pass in one call, which overlaps them where the shape allows."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    dev = q.device
    saved = torch.empty((_lib.size("kdn_mem_saved_size", B, T, H, K, V),), device=dev, dtype=torch.uint8)
    o = torch.empty((B, T, H, V), device=dev, dtype=out_dtype)
    ht = torch.empty((B, H, K, V), device=dev, dtype=torch.float32) if output_final_state else None
    h0 = initial_state.float().contiguous() if initial_state is not None else None
    stream = _lib.stream_of(q)
    extra = 0 if need_backward else NO_BACKWARD
    if overlap is None:
        overlap = DEFAULT_OVERLAP and not _lib.timing()
    for bit, tag in (FWD_STAGES_OVERLAP if overlap else FWD_STAGES):
        _lib.call("kdn_mem_fwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(kappa_or_beta), int(iso), _lib.ptr(v),
                  _lib.ptr(g_cumsum), B, T, H, K, V, float(scale), _lib.ptr(h0), _lib.ptr(saved), saved.numel(),
                  _lib.ptr(ht), _lib.ptr(o), _lib.is_bf16(o), _lib.ptr(q_rstd), _lib.ptr(k_rstd), bit | extra,
                  stream, tag=tag)
    return o, saved, ht


def rebuild_saved(q, k, kappa_or_beta, iso: bool, v, g_cumsum, scale: float, *, initial_state=None,
                  fused_norm=False):
    """The buffer mem_fwd(need_backward=True) returns as ``saved``, rebuilt from the op's inputs for
    mem_bwd (the "recompute" backward mode): the intra-chunk build (stage bit 0) and the serial state
    pass without the readout (bit 1), on the same kernels as the forward, so every intermediate is
    bit-identical to the forward's.  With ``fused_norm`` q and k are the raw inputs of the in-op L2
    norm; the rows' rstd it writes again go to scratch (the forward's are the ones mem_bwd takes)."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    dev = q.device
    saved = torch.empty((_lib.size("kdn_mem_saved_size", B, T, H, K, V),), device=dev, dtype=torch.uint8)
    h0 = initial_state.float().contiguous() if initial_state is not None else None
    rs = torch.empty((2, B, T, H), device=dev, dtype=torch.float32) if fused_norm else None
    stream = _lib.stream_of(q)
    for bit, tag in ((1, "mem_intra_fwd"), (2, "mem_state_fwd")):
        _lib.call("kdn_mem_fwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(kappa_or_beta), int(iso), _lib.ptr(v),
                  _lib.ptr(g_cumsum), B, T, H, K, V, float(scale), _lib.ptr(h0), _lib.ptr(saved), saved.numel(),
                  None, None, 0, _lib.ptr(rs[0]) if fused_norm else None,
                  _lib.ptr(rs[1]) if fused_norm else None, bit, stream, tag=tag)
    return saved


def mem_bwd(q, k, kappa_or_beta, iso: bool, v, g_cumsum, saved, scale: float, do, *, d_final_state=None,
            need_initial_state_grad=False, q_rstd=None, k_rstd=None, overlap=None):
    """Returns (dq bf16, dk bf16, dv bf16, dkappa f32 [B,T,H,K] or dbeta f32 [B,T,H],
    dg f32 natural-log not reverse-summed, d_initial_state or None).

    ``overlap`` (default: unless a KernelTimer is timing each kernel) launches the reverse pass and
    the chunk backward in one call, which overlaps them where the shape allows.

    With ``q_rstd`` / ``k_rstd`` [B,T,H] (the in-op L2 norm, as mem_fwd wrote them) q and k are the
    raw bf16 inputs the forward normalised, and dq, dk are the gradients of the raw inputs."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    dev = q.device
    ws = torch.empty((_lib.size("kdn_mem_bwd_workspace_size", B, T, H, K, V),), device=dev, dtype=torch.uint8)
    dq = torch.empty((B, T, H, K), device=dev, dtype=torch.bfloat16)
    dk = torch.empty_like(dq)
    dv = torch.empty((B, T, H, V), device=dev, dtype=torch.bfloat16)
    dkap = torch.empty((B, T, H) if iso else (B, T, H, K), device=dev, dtype=torch.float32)
    dg = torch.empty((B, T, H, K), device=dev, dtype=torch.float32)
    dh0 = torch.empty((B, H, K, V), device=dev, dtype=torch.float32) if need_initial_state_grad else None
    dht = d_final_state.float().contiguous() if d_final_state is not None else None
    if do.dtype not in (torch.bfloat16, torch.float32):
        do = do.float()
    do = do.contiguous()
    stream = _lib.stream_of(q)
    if overlap is None:
        overlap = DEFAULT_OVERLAP and not _lib.timing()
    for bit, tag in (BWD_STAGES_OVERLAP if overlap else BWD_STAGES):
        _lib.call("kdn_mem_bwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(kappa_or_beta), int(iso), _lib.ptr(g_cumsum),
                  B, T, H, K, V, float(scale), _lib.ptr(do), _lib.is_bf16(do), _lib.ptr(dht), _lib.ptr(saved),
                  saved.numel(), _lib.ptr(ws), ws.numel(), _lib.ptr(dq), _lib.ptr(dk),
                  None if iso else _lib.ptr(dkap), _lib.ptr(dkap) if iso else None, _lib.ptr(dv), _lib.ptr(dg),
                  _lib.ptr(dh0), _lib.ptr(q_rstd), _lib.ptr(k_rstd), bit, stream, tag=tag)
    return dq, dk, dv, dkap, dg, dh0
