#!/usr/bin/env python
"""Benchmark of the KDN mixer scan on one MI355X (BASELINE.json metric).

A step is one forward + backward of the KDN mixer scan of one layer (gate/frontend ->
Kalman gain -> chunked memory scan, gradients for every input and parameter) at
B=4, H=18, T=4096, d_k=d_v=128, bf16 inputs with fp32 state, on synthetic data resident
in HBM.  The headline line is iso_kdn; the diag_kdn figure (config 2)
is reported alongside under "also".  Kernels are timed with HIP events recorded on their
launch stream inside the timed region; the dominant kernel's roofline is reported against
MI355X peaks.  The CPU baseline times the oracle's tokenwise recurrence (fp32, autograd)
on a bounded sample of (b, h) slices on the host cores.

  python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--variant iso|diag] [--cpu-slices 8]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "kalman-delta-networks_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "KDN mixer fwd+bwd tokens/s at B4 H18 T4096 d128 bf16; % MFMA/HBM peak"
HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3   # dense fp32 MFMA (v_mfma_f32_16x16x4_f32)
BF16_PEAK_TFLOPS = 2500.0  # dense bf16 MFMA
C = 64
# minimum I/O of the whole mixer scan op per token-head (inputs read once, outputs written once):
# iso fwd 1,544 + bwd 2,832; diag fwd 2,052 + bwd 3,848 (d = 128)
OP_BYTES = {"iso": lambda d: (6 * d + 4 * d + 8 + 2 * d) + (22 * d + 16),
            "diag": lambda d: (6 * d + 4 * d + 4 * d + 4 + 2 * d) + (30 * d + 8)}
OP_FWD_BYTES = {"diag": lambda d: 6 * d + 4 * d + 4 * d + 4 + 2 * d}
# calibrated counter traffic per variant (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs of this script)
TRAFFIC_FILES = [os.path.join(ROOT, "profiles", f) for f in ("kdn_traffic.json", "kdn_traffic_diag.json")]

# MFMA path of each kernel: "f32" = fp32 MFMA; "bf16x3" = fp32-grade products as three bf16
# MFMAs (hi*hi + hi*lo + lo*hi), whose ceiling is the bf16 peak / 3 in algorithmic FLOP/s.
MFMA_PATH = {"mem_intra_fwd": "bf16x3", "mem_state_readout_fwd": "bf16x3",
             "mem_state_bwd": "bf16x3", "mem_bwd_chunk": "bf16x3"}


def mfma_peak(tag: str) -> float:
    return FP32_PEAK_TFLOPS if MFMA_PATH.get(tag, "f32") == "f32" else BF16_PEAK_TFLOPS / 3.0


def kernel_counts(variant: str, B: int, T: int, H: int, K: int, V: int, infer: bool = False,
                  half_states: bool = False):
    """Algorithmic HBM bytes and FLOPs per launch of each kernel (inputs read once, outputs
    written once, no recompute).  N = B*T*H token-heads; per-token-head figures times N.  With
    ``infer`` (no backward follows) the forward kernels skip what only the backward reads: A^T, and
    h and delta of the fused state pass.  ``half_states``: the per-chunk state copies h and dh the
    backward reads are bf16 (the isotropic scan with one chunk group)."""
    N = B * T * H
    kap_in = 4 * K if variant == "diag" else 4           # kappa fp32 [K] or beta fp32
    dkap_out = 4 * K if variant == "diag" else 4
    do_b = 4 * V if variant == "diag" else 2 * V         # diag output cotangent is fp32
    h_b = (2 if half_states else 4) * K * V / C           # one state copy per chunk
    mm = C * C / C * 4                                    # one fp32 C x C matrix per chunk
    per = {
        # q,k,v bf16 + kappa + g fp32 -> U, W, Kf, Qg fp32 + M, A^T (the inverse, saved)
        # (iso: q, k raw, normalised in the kernel, and their rows' rstd written)
        "mem_intra_fwd": (2 * 2 * K + 2 * V + kap_in + 4 * K + 4 * (V + 3 * K) + 2 * mm
                          + (8 if variant == "iso" else 0),
                          2 * (C * K + C * (V + K) / 2)),
        # U, W, Kf, g_last, Qg, M -> h, delta, o  (one chunk group: the state pass does the readout)
        "mem_state_readout_fwd": (4 * V + 8 * K + 4 * K / C + h_b + 4 * V + 4 * K + mm
                                  + (2 if variant == "iso" else 4) * V,
                                  2 * 2 * K * V + 2 * (K * V + C * V / 2)),
        # M, Kf, Qg, W, dO -> dh, d delta
        "mem_state_bwd": (mm + 12 * K + do_b + h_b + 4 * V, 2 * (C * V / 2 + 3 * K * V)),
        # h, dh, delta, d delta, dO, A^T, U, W, q, k, kappa, g (iso: and the q / k rstd of the in-op norm,
        # whose backward it applies) -> dv, dq, dk, dkappa, dg (dQg, dW, dKf, dM, dKg and dN stay on chip);
        # FLOPs: the state-gradient products, the solves and dN, the gradient contractions
        "mem_bwd_chunk": (2 * h_b + 8 * V + do_b + mm + 4 * V + 4 * K + 2 * 2 * K + kap_in + 4 * K
                          + 2 * V + 2 * 2 * K + dkap_out + 4 * K + (8 if variant == "iso" else 0),
                          2 * (3 * K * V + C * V / 2) + 2 * (C * (V + K) / 2 + C * (V + K) / 2) + 2 * 2 * (C * K)),
    }
    if infer:
        b, f = per["mem_intra_fwd"]
        per["mem_intra_fwd"] = (b - mm, f)
        b, f = per["mem_state_readout_fwd"]
        per["mem_state_readout_fwd"] = (b - h_b - 4 * V, f)
    return {k: (b * N, f * N) for k, (b, f) in per.items()}


def frontend_counts(variant: str, B: int, T: int, H: int, K: int):
    """Algorithmic HBM bytes per call of the gate / gain / norm entry points around the memory
    scan (inputs read once, outputs written once; no FLOP bound).  N = B*T*H token-heads,
    E = N*K elements.  ``l2norm_*`` is one tensor per call (q and k: two calls per step)."""
    N = B * T * H
    E = N * K
    if variant == "iso":
        per = {
            # the scan's gate -> gain runs fused (lit_gpt/kdn_ops/iso_kdn_chunk.py iso_kdn_front):
            # g_raw bf16, omega|r raw bf16 -> g_cumsum f32, a, omega, r, beta, p_prev f32 (a, omega, r, p_prev
            # saved for the backward)
            "iso_front_fwd": 6 * E + 28 * N,
            # g_raw, omega|r raw, dg f32, dbeta, a, omega, r, p_prev -> dg_raw bf16, d omega|r raw bf16
            # (the cotangents of a, omega, r stay on chip)
            "iso_front_bwd": 8 * E + 28 * N,
            # the two ops called separately:
            # g_raw bf16, omega|r raw bf16 -> g_cumsum f32, a, omega, r f32
            "iso_gate_fwd": 6 * E + 16 * N,
            # g_raw, omega|r raw, dg f32, da, domega, dr -> dg_raw bf16, d omega|r raw bf16
            "iso_gate_bwd": 8 * E + 20 * N,
            # a, omega, r -> beta, p_prev
            "iso_gain_fwd": 20 * N,
            # a, omega, r, dbeta, p_prev -> da, domega, dr
            "iso_gain_bwd": 32 * N,
            # x bf16 -> y bf16, rstd f32
            "l2norm_fwd": 4 * E + 4 * N,
            # x bf16, rstd, dy bf16 -> dx bf16
            "l2norm_bwd": 6 * E + 4 * N,
        }
    else:
        # the scan's front half runs fused (normalisation -> frontend -> gain, lit_gpt/kdn_ops/diag_kdn_chunk.py
        # diag_kdn_front): alpha, omega, r and the fp32 gain key never reach HBM
        per = {
            # q, k bf16 -> q_memory, k_memory bf16, two norms
            "diag_front_norm_fwd": 8 * E + 8 * N,
            # k bf16, k norm, retention, omega raw bf16, r raw bf16 -> g_cumsum, kappa f32
            "diag_front_fwd": 16 * E + 6 * N,  # with the even tokens' precisions saved for the backward
            # k, k norm, retention, omega raw, r raw, d g_cumsum, d kappa f32, d k_memory bf16
            #   -> dk, d retention raw, d omega raw bf16, d r raw
            "diag_front_bwd": 24 * E + 8 * N,  # ... which it reads
            # q bf16, q norm, d q_memory bf16 -> dq bf16
            "diag_front_norm_bwd": 6 * E + 4 * N,
        }
    return {k: (b, 0) for k, b in per.items()}


# The scope's own per-unit figures for the kernels it prices (per token-head, d = K = V, C = 64):
# the chunk backward carries the whole backward's minimum I/O (iso 22d+16, diag 30d+8), the state pass
# reads w, u, kg and writes v_new plus one state per chunk (16d + 4d^2/C).  A kernel the scope gives
# no byte figure for falls back to its decomposition bytes.
S8D_BYTES = {"mem_bwd_chunk": {"iso": lambda d: 22 * d + 16, "diag": lambda d: 30 * d + 8},
             "mem_state_readout_fwd": {"iso": lambda d: 16 * d + 4 * d * d / C,
                                       "diag": lambda d: 16 * d + 4 * d * d / C}}


def headline_roofline(variant: str, tag: str, kern: dict, B: int, T: int, H: int, K: int, traffic=(None, None)):
    """The dominant kernel against MI355X's HBM peak, priced on the scope's algorithmic bytes for it
    (S8D_BYTES per token-head times B*T*H) over its mean event-timed duration; the figure on this
    decomposition's own bytes (kernel_counts) is kept beside it."""
    t = kern["ms"] * 1e-3
    per = S8D_BYTES.get(tag, {}).get(variant)
    nbytes_traffic, source = traffic
    out = {"kernel": tag, "bound": "hbm", "peak": HBM_PEAK_GBS, "unit": "GB/s", "traffic": nbytes_traffic,
           "traffic_source": (os.path.relpath(source, ROOT) if source is not None else None),
           "kernel_ms": kern["ms"]}
    if per is not None:
        nbytes = per(K) * B * T * H
        out.update(achieved=round(nbytes / t / 1e9, 2), frac=round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4),
                   alg_bytes=int(nbytes), bytes_per_token_head=per(K),
                   basis="scope minimum bytes (backward minimum for the chunk backward)")
    else:
        out.update(achieved=kern["achieved"], frac=kern["frac"], alg_bytes=kern["alg_bytes"],
                   basis="decomposition bytes")
    out["decomposition"] = {"alg_bytes": kern["alg_bytes"], "achieved": kern["achieved"], "frac": kern["frac"],
                            "note": "this build's own reads and writes for the kernel (inputs once, outputs once)"}
    return out


def op_roofline(variant: str, ms: float, B: int, T: int, H: int, K: int):
    """The whole op against its HBM floor: the minimum I/O bytes of the mixer scan fwd+bwd (OP_BYTES per
    token-head times B*T*H) over the measured step time."""
    nbytes = OP_BYTES[variant](K) * B * T * H
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "bytes_per_token_head": OP_BYTES[variant](K), "alg_bytes": int(nbytes),
            "ceiling_ms": round(nbytes / (HBM_PEAK_GBS * 1e9) * 1e3, 4), "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}


def run_variant(variant: str, steps: int, warmup: int, B: int, T: int, H: int, K: int):
    import torch

    from lit_gpt.kdn_ops import _lib, _memscan
    from lit_gpt.kdn_ops.scan import diag_kdn_scan, iso_kdn_scan
    from lit_gpt.kdn_ops.synthetic import GRAD_KEYS, make_inputs

    dev = torch.device("cuda:0")
    inputs, do = make_inputs(variant, B, T, H, K, seed=0, device=dev)
    leaves = {k: x.requires_grad_(True) for k, x in inputs.items()}
    keys = [k for k in GRAD_KEYS[variant]]
    fn = iso_kdn_scan if variant == "iso" else diag_kdn_scan

    def step():
        o = fn(**leaves)
        grads = torch.autograd.grad(o, [leaves[k] for k in keys], grad_outputs=do)
        return grads

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # the step rate is timed without per-call events; a second pass of the same steps times each
    # entry point with HIP events on its launch stream
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / steps
    with _lib.KernelTimer() as timer:
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
    kernel_ms = {tag: timer.mean_ms(tag) for tag in timer.tags()}
    half = variant == "iso" and _memscan.state_groups(B, T, H, K, K) == 1
    counts = kernel_counts(variant, B, T, H, K, K, half_states=half)
    counts.update(frontend_counts(variant, B, T, H, K))
    per_kernel = {}
    for tag, (nbytes, flops) in counts.items():
        if tag not in kernel_ms:  # an entry point this shape does not call (e.g. the separate readout when fused)
            continue
        t = kernel_ms[tag] * 1e-3
        t_hbm = nbytes / (HBM_PEAK_GBS * 1e9)
        t_mfma = flops / (mfma_peak(tag) * 1e12)
        bound = "hbm" if t_hbm >= t_mfma else "mfma"
        if bound == "hbm":
            achieved, peak, unit = nbytes / t / 1e9, HBM_PEAK_GBS, "GB/s"
        else:
            achieved, peak, unit = flops / t / 1e12, round(mfma_peak(tag), 1), "TFLOP/s"
        per_kernel[tag] = dict(ms=round(t * 1e3, 4), bound=bound, achieved=round(achieved, 2), peak=peak,
                               unit=unit, frac=round(achieved / peak, 4), mfma=MFMA_PATH.get(tag, "f32"),
                               alg_bytes=int(nbytes), alg_flops=int(flops))
        if tag in MFMA_PATH:  # the MFMA view beside the binding one: algorithmic FLOP/s against the path peak
            per_kernel[tag]["mfma_tflops"] = round(flops / t / 1e12, 2)
            per_kernel[tag]["mfma_frac"] = round(flops / t / 1e12 / mfma_peak(tag), 4)
    dominant = max(per_kernel, key=lambda k: per_kernel[k]["ms"])
    return dict(ms_per_step=ms, tokens_per_s=B * T / (ms * 1e-3), kernels=per_kernel, dominant=dominant)


def run_layer_frontends(steps: int, warmup: int, B: int, T: int, H: int, K: int):
    """Layer frontends around the scan at the same shape: the packed q|k|v short convolution
    (x [B,T,3HK] bf16) and the gated output norm (o, gate [B,T,H,K] bf16), fwd+bwd, timed per
    kernel launch; HBM-bound, priced at their minimum bytes."""
    import torch

    from lit_gpt.kdn_ops import _lib
    from lit_gpt.kdn_ops.gated_norm import FusedRMSNormGated
    from lit_gpt.kdn_ops.short_conv import qkv_causal_conv1d

    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(1)
    D = H * K
    x = torch.randn(B, T, 3 * D, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    w = (0.5 * torch.randn(3 * D, 4, generator=g)).to(torch.bfloat16).to(dev).requires_grad_(True)
    dqkv = [torch.randn(B, T, D, generator=g).to(torch.bfloat16).to(dev) for _ in range(3)]
    o = torch.randn(B, T, H, K, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    gate = torch.randn(B, T, H, K, generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    do = torch.randn(B, T, H, K, generator=g).to(torch.bfloat16).to(dev)
    norm = FusedRMSNormGated(K, activation="sigmoid", eps=1e-5).to(dev)

    def step():
        outs = qkv_causal_conv1d(x, w)
        torch.autograd.grad(outs, (x, w), dqkv)
        y = norm(o, gate)
        torch.autograd.grad(y, (o, gate, norm.weight), do)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    with _lib.KernelTimer() as timer:
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
    N = B * T * D
    nbytes = {"short_conv_fwd": 2 * N * 2, "short_conv_bwd": 3 * N * 2,  # per q|k|v group launch
              "rms_norm_gated_fwd": 3 * N * 2 + B * T * H * 4, "rms_norm_gated_bwd": 5 * N * 2 + B * T * H * 4}
    out = {}
    for tag, nb in nbytes.items():
        t = timer.mean_ms(tag) * 1e-3
        achieved = nb / t / 1e9
        out[tag] = dict(ms=round(t * 1e3, 4), bound="hbm", achieved=round(achieved, 2), peak=HBM_PEAK_GBS,
                        unit="GB/s", frac=round(achieved / HBM_PEAK_GBS, 4), alg_bytes=int(nb))
    return out


def run_config4(name: str, steps: int, warmup: int, B: int, T: int):
    """The whole random-init config-4 model (``name``, mamba init) on synthetic token ids.

    * forward (the config-4 workload): bf16 weights, eval mode, no autograd; logits over the
      padded vocabulary.  The KDN-mixer share is one mixer layer's forward at the same shape,
      timed alone, times the layer count, over the model's forward time.
    * training step (reported beside it): fp32 master weights, forward under CUDA bf16 autocast,
      the fused cross-entropy on the bf16 logits (``FusedCrossEntropyLoss``, as the reference's
      pretrain.py:1165,1258 applies it), backward, fused AdamW; mixer share from one mixer
      layer's fwd+bwd alone.
    * the cross-entropy kernels alone on [B*T, vocab] bf16 logits, each in its own loop, timed
      with HIP events, with their HBM fraction (forward reads the logits once; backward reads
      them and writes the gradient).
    """
    import torch

    from lit_gpt.fused_cross_entropy import FusedCrossEntropyLoss
    from lit_gpt.kdn_ops import _lib
    from lit_gpt.model import GPT

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    with torch.device(dev):
        model = GPT.from_name(name)
    model.init_weights()
    cfg = model.config
    V = cfg.padded_vocab_size
    idx = torch.randint(0, cfg.vocab_size, (B, T + 1), device=dev)
    x = torch.randn(B, T, cfg.n_embd, device=dev, requires_grad=True)
    dy = torch.randn(B, T, cfg.n_embd, device=dev, dtype=torch.bfloat16)
    mixer = model.transformer.h[0].attn

    def timed(fn, n, w):
        for _ in range(w):
            fn()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(n):
            fn()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / n

    # training step
    model.train()
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4, weight_decay=0.1, fused=True)
    loss_fn = FusedCrossEntropyLoss()

    def train_step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits = model(idx[:, :-1])
        loss = loss_fn(logits, idx[:, 1:])
        loss.backward()
        opt.step()
        opt.zero_grad(set_to_none=True)

    def mixer_fwd_bwd():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out = mixer(x)[0]
        torch.autograd.grad(out, [x] + list(mixer.parameters()), dy)

    train_ms = timed(train_step, steps, warmup)
    mixer_train_ms = timed(mixer_fwd_bwd, steps, warmup)
    del opt
    torch.cuda.empty_cache()

    # forward (config 4)
    model = model.to(torch.bfloat16).eval()
    xb = x.detach().to(torch.bfloat16)

    @torch.no_grad()
    def forward():
        model(idx[:, :-1])

    @torch.no_grad()
    def mixer_fwd():
        mixer(xb)

    fwd_ms = timed(forward, steps, warmup)
    mixer_fwd_ms = timed(mixer_fwd, steps, warmup)
    del model
    torch.cuda.empty_cache()

    # cross-entropy kernels alone, each in a steady-state loop of its own (forward repeatedly,
    # then backward into one gradient buffer), so neither pays for another kernel's write-back
    from lit_gpt.fused_cross_entropy import xent_backward, xent_forward
    n = B * T
    logits = torch.randn(n, V, device=dev, dtype=torch.bfloat16).mul_(4)
    labels = idx[:, 1:].reshape(-1)
    dlogits = torch.empty_like(logits)
    dloss = torch.full((n,), 1.0 / n, device=dev)
    _, lse, _ = xent_forward(logits, labels)
    reps = max(steps, 10)
    xent_us = {}
    for tag, fn in (("xent_fwd", lambda: xent_forward(logits, labels)),
                    ("xent_bwd", lambda: xent_backward(dloss, logits, lse, labels, dlogits=dlogits))):
        timed(fn, 2, 2)
        with _lib.KernelTimer() as kt:
            for _ in range(reps):
                fn()
            xent_us[tag] = kt.mean_ms(tag) * 1e3
    del logits, dlogits
    torch.cuda.empty_cache()
    xent_bytes = {"xent_fwd": n * V * 2 + n * 8 + 3 * n * 4, "xent_bwd": 2 * n * V * 2 + n * 8 + 2 * n * 4}
    xent_rep = {}
    for tag, us in xent_us.items():
        gbs = xent_bytes[tag] / (us * 1e-6) / 1e9
        xent_rep[tag] = {"us": round(us, 2), "alg_bytes": int(xent_bytes[tag]), "achieved_GBps": round(gbs, 1),
                         "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
    L = cfg.n_layer
    return {"workload": f"{name} forward, random init (mamba), bf16 weights, synthetic token ids, logits over "
                        f"{V}; training step beside it",
            "B": B, "T": T, "n_layer": L, "value": round(B * T / (fwd_ms * 1e-3), 1), "unit": "tokens/s",
            "ms_per_forward": round(fwd_ms, 3), "mixer_layer_fwd_ms": round(mixer_fwd_ms, 3),
            "mixer_share": round(L * mixer_fwd_ms / fwd_ms, 4),
            "cross_entropy_kernels": {"shape": [n, V], "dtype": "bf16", **xent_rep},
            "train_step": {"what": "fwd (bf16 autocast, fp32 master weights) + fused cross-entropy on the bf16 "
                                   "logits + bwd + fused AdamW",
                           "value": round(B * T / (train_ms * 1e-3), 1), "unit": "tokens/s",
                           "ms_per_step": round(train_ms, 3), "mixer_layer_fwd_bwd_ms": round(mixer_train_ms, 3),
                           "mixer_share": round(L * mixer_train_ms / train_ms, 4)}}


def run_decode(name: str, steps: int, warmup: int, prompt: int = 1024):
    """Token-by-token decoding of the random-init config-4 model (bf16 weights, eval) after a
    ``prompt``-token prefill, eager and as a replayed HIP graph (``KDNDecoder``), at batch 1 and 32:
    ms per decode step (one token for each of B sequences) and tokens/s = B / step time.  Beside it,
    the single-token kernels alone at the model's H18 d128 and B in {1, 64}: ``kdn_mem_step``
    (memory only) and ``kdn_kalman_step`` (the iso gain from the carried precision + memory, the
    kernel the model's decode runs); HBM-bound, algorithmic bytes = B H (2 K V 4 state read +
    write, q, k, v, o bf16, g f32, and beta or a, omega, r, precision in and out)."""
    import torch

    from lit_gpt.decode import KDNDecoder
    from lit_gpt.kdn_ops import _lib
    from lit_gpt.kdn_ops.step import kdn_kalman_step, kdn_memory_step
    from lit_gpt.fused_cross_entropy import FusedCrossEntropyLoss
    from lit_gpt.kdn_ops import _lib
    from lit_gpt.model import GPT

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    with torch.device(dev):
        model = GPT.from_name(name)
    model.init_weights()
    model = model.to(torch.bfloat16).eval()
    cfg = model.config
    H, K = cfg.n_head, cfg.head_size

    def timed(fn, n, w):
        for _ in range(w):
            fn()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(n):
            fn()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / n

    out = {"workload": f"{name} decode after a {prompt}-token prefill, bf16 weights, random init, synthetic ids",
           "unit": "tokens/s", "model": {}}
    for B in (1, 32):
        idx = torch.randint(0, cfg.vocab_size, (B, prompt), device=dev)
        row = {}
        for use_graph in (False, True):
            dec = KDNDecoder(model, B, use_graph=use_graph)
            dec.prefill(idx)
            tok = idx[:, -1].clone()
            ms = timed(lambda: dec.step(tok), steps, warmup)
            row["graph" if use_graph else "eager"] = {"ms_per_step": round(ms, 4), "value": round(B / (ms * 1e-3), 1)}
            del dec
        out["model"][f"B{B}"] = row
    del model
    torch.cuda.empty_cache()
    kern, kal = {}, {}
    for B in (1, 64):
        g = torch.Generator(device=dev).manual_seed(B)
        q = torch.randn(B, 1, H, K, device=dev, generator=g).bfloat16()
        k = torch.randn(B, 1, H, K, device=dev, generator=g).bfloat16()
        v = torch.randn(B, 1, H, K, device=dev, generator=g).bfloat16()
        gc = (-0.1 * torch.rand(B, 1, H, K, device=dev, generator=g)).float()
        beta = torch.rand(B, 1, H, device=dev, generator=g)
        a, w, r = (0.5 + torch.rand(B, 1, H, device=dev, generator=g) for _ in range(3))
        prec = [torch.ones(B, H, device=dev), torch.empty(B, H, device=dev)]
        S = torch.zeros(B, H, K, K, device=dev)
        for _ in range(warmup):
            kdn_memory_step(q, k, v, gc, state=S, beta=beta)
            kdn_kalman_step(q, k, v, gc, state=S, precision=prec[0], precision_out=prec[1], a=a, omega=w, r=r,
                            info_scale=float(K))
        with _lib.KernelTimer() as kt:
            for i in range(steps):
                kdn_memory_step(q, k, v, gc, state=S, beta=beta)
                kdn_kalman_step(q, k, v, gc, state=S, precision=prec[i % 2], precision_out=prec[1 - i % 2], a=a,
                                omega=w, r=r, info_scale=float(K))
        for tag, extra, dst in (("mem_step", 4, kern), ("kalman_step", 5 * 4, kal)):
            ms = kt.mean_ms(tag)
            alg = B * H * (2 * K * K * 4 + 3 * K * 2 + K * 4 + extra + K * 2)
            gbs = alg / (ms * 1e-3) / 1e9
            dst[f"B{B}"] = {"us": round(ms * 1e3, 2), "alg_bytes": alg, "achieved_GBps": round(gbs, 1),
                            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
    out["mem_step_kernel"] = kern
    out["kalman_step_kernel"] = kal
    return out


def cpu_baseline(variant: str, slices: int, T: int, K: int, B: int, H: int):
    """Oracle tokenwise recurrence (fp32, torch autograd) fwd+bwd on `slices` (b, h) slices."""
    import torch

    from lit_gpt.kdn_ops.synthetic import GRAD_KEYS, make_inputs
    from oracle import kdn_oracle as ko

    torch.set_num_threads(os.cpu_count() or 1)
    names = {"q": "q_raw", "k": "k_raw", "initial_precision_param": "mu_param"}
    mixer = ko.iso_mixer if variant == "iso" else ko.diag_mixer
    t_total = 0.0
    for s in range(slices):
        inputs, do = make_inputs(variant, 1, T, 1, K, seed=100 + s, device="cpu", dtype=torch.float32)
        leaves = {k: x.requires_grad_(True) for k, x in inputs.items()}
        t0 = time.perf_counter()
        o = mixer(**{names.get(k, k): x for k, x in leaves.items()})
        torch.autograd.grad(o, [leaves[k] for k in GRAD_KEYS[variant]], grad_outputs=do)
        t_total += time.perf_counter() - t0
    per_slice = t_total / slices
    tokens_per_s = B * T / (per_slice * B * H)
    return dict(value=round(tokens_per_s, 2), unit="tokens/s", cores=torch.get_num_threads(), kind="port",
                sample=f"{slices} of {B * H} (b,h) slices at T={T}, d={K}: oracle tokenwise fp32 fwd+bwd "
                       f"(autograd), {per_slice:.2f} s/slice, extrapolated to the {B}x{H} job")


def run_config3(steps: int, warmup: int, B: int = 1, T: int = 32768, H: int = 18, K: int = 128):
    """the diag mixer scan forward at B1 H18 T32768 d128 (bf16 inputs) from a carried
    state: S0 ~ N(0, 0.02^2) fp32 [B,H,K,V] and a per-channel initial precision softplus(N(0,1))
    [B,H,K] (the oracle's initial_precision, diag_kdn_naive.py:503-516), returning the final memory and
    precision.  Forward only, no autograd.  The op's minimum HBM bytes are 2,052 per token-head plus
    the state and precision read and written; the per-kernel fractions use the kernels' own
    algorithmic bytes at this shape."""
    import torch

    from lit_gpt.kdn_ops import _lib
    from lit_gpt.kdn_ops.scan import diag_kdn_scan
    from lit_gpt.kdn_ops.synthetic import make_inputs

    dev = torch.device("cuda:0")
    inputs, _ = make_inputs("diag", B, T, H, K, seed=0, device=dev)
    g = torch.Generator().manual_seed(3)
    S0 = (0.02 * torch.randn(B, H, K, K, generator=g)).to(dev)
    P0 = torch.nn.functional.softplus(torch.randn(B, H, K, generator=g)).to(dev)

    @torch.no_grad()
    def step():
        return diag_kdn_scan(**inputs, initial_state=S0, initial_precision=P0, output_final_state=True)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    with _lib.KernelTimer() as timer:
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
    fwd_tags = ("diag_front_norm_fwd", "diag_front_fwd", "mem_intra_fwd", "mem_state_readout_fwd")
    counts = kernel_counts("diag", B, T, H, K, K, infer=True)
    counts.update(frontend_counts("diag", B, T, H, K))
    kernels = {}
    for tag in fwd_tags:
        nbytes, _fl = counts[tag]
        if tag == "mem_state_readout_fwd":  # the long-context output is bf16 (v's dtype), not the fp32 of kernel_counts
            nbytes -= 2 * K * B * T * H
        t = timer.mean_ms(tag) * 1e-3
        gbs = nbytes / t / 1e9
        kernels[tag] = {"ms": round(t * 1e3, 4), "bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "alg_bytes": int(nbytes)}
    N = B * T * H
    op_bytes = OP_FWD_BYTES["diag"](K) * N + 2 * (B * H * K * K * 4 + B * H * K * 4)
    dominant = max(kernels, key=lambda k: kernels[k]["ms"])
    return {"workload": "diag_kdn mixer scan forward from a carried state (S0 ~ N(0, 0.02^2), per-channel "
                        "precision softplus(N(0,1))), returning the final memory and precision",
            "B": B, "T": T, "H": H, "d": K, "inputs": "bf16", "state": "fp32",
            "value": round(B * T / (ms * 1e-3), 1), "unit": "tokens/s", "ms_per_forward": round(ms, 4),
            "op_roofline": {"bound": "hbm", "alg_bytes": int(op_bytes), "ceiling_ms": round(op_bytes / 8e12 * 1e3, 4),
                            "achieved": round(op_bytes / (ms * 1e-3) / 1e9, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(op_bytes / (ms * 1e-3) / 8e12, 4)},
            "dominant": dominant, "kernels": kernels}


def cpu_baseline_config3(T: int, K: int, B: int, H: int):
    """The oracle's diag mixer forward (fp32: tokenwise gain, WY-chunked memory) from a carried state on
    one (b, h) slice of the config-3 workload, extrapolated to the B x H job."""
    import torch

    from lit_gpt.kdn_ops.synthetic import make_inputs
    from oracle import kdn_oracle as ko

    torch.set_num_threads(os.cpu_count() or 1)
    inputs, _ = make_inputs("diag", 1, T, 1, K, seed=100, device="cpu", dtype=torch.float32)
    g = torch.Generator().manual_seed(3)
    S0 = 0.02 * torch.randn(1, 1, K, K, generator=g)
    P0 = torch.nn.functional.softplus(torch.randn(1, 1, K, generator=g))
    names = {"q": "q_raw", "k": "k_raw", "initial_precision_param": "mu_param"}
    t0 = time.perf_counter()
    with torch.no_grad():
        ko.diag_mixer(**{names.get(k, k): x for k, x in inputs.items()}, chunked=True, gain_chunked=False,
                      initial_state=S0, initial_precision=P0, output_final_state=True)
    per_slice = time.perf_counter() - t0
    return dict(value=round(B * T / (per_slice * B * H), 2), unit="tokens/s", cores=torch.get_num_threads(),
                kind="port", sample=f"1 of {B * H} (b,h) slices at T={T}, d={K}: oracle diag mixer forward "
                                    f"(fp32, WY-chunked memory) from a carried state, {per_slice:.2f} s/slice, "
                                    f"extrapolated to the {B}x{H} job")


def measured_traffic(kernel: str, config: str):
    """(HBM bytes per launch of `kernel`, the file they come from) from the committed rocprofv3 --pmc summary
    whose config is `config` (FETCH_SIZE + WRITE_SIZE, each scaled by the copy-kernel calibration), or (None, None)."""
    for path in TRAFFIC_FILES:
        try:
            with open(path) as f:
                rec = json.load(f)
        except (OSError, ValueError):
            continue
        k = rec.get("kernels", {}).get(kernel)
        if rec.get("config") == config and k:
            return int(k["fetch_bytes"] + k["write_bytes"]), path
    return None, None


def calib_copy(mib: int):
    """A plain device copy of known size, for calibrating FETCH_SIZE / WRITE_SIZE."""
    import torch

    x = torch.ones(mib * (1 << 20) // 4, device="cuda:0")
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()


def _lib_size(name: str, *dims) -> int:
    from lit_gpt.kdn_ops import _lib
    return int(_lib.size(name, *dims))


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--variant", choices=("iso", "diag"), default="iso")
    ap.add_argument("--cpu-slices", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-config4", action="store_true", help="skip the whole-model (config 4) measurement")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode (state-carry) measurement")
    ap.add_argument("--decode-only", action="store_true", help="measure only decoding and print its line")
    ap.add_argument("--no-config3", action="store_true", help="skip the long-context (config 3) measurement")
    ap.add_argument("--config3-only", action="store_true",
                    help="measure only the long-context diag forward (config 3) and print its line")
    ap.add_argument("--config4-only", action="store_true",
                    help="measure only the whole model (config 4) and print its line (for profiling)")
    ap.add_argument("--headline-only", action="store_true",
                    help="time only the main variant's step and print its line (for profiling)")
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="also run a plain copy of MIB MiB (PMC byte-counter calibration)")
    ap.add_argument("--serial-schedule", action="store_true",
                    help="launch every memory-scan kernel in its own call, no overlapped segments (for a "
                         "profiler that averages per-kernel durations, as the bench's event-timed pass does)")
    ap.add_argument("--backward-mode", choices=("save", "recompute"), default="save",
                    help="what the memory scan's forward keeps for the backward (the headline uses 'save'; "
                         "the full run reports 'recompute' beside it under also.recompute_backward)")
    ap.add_argument("--B", type=int, default=4)
    ap.add_argument("--T", type=int, default=4096)
    ap.add_argument("--H", type=int, default=18)
    ap.add_argument("--d", type=int, default=128)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build runs the KDN scan on a single GPU "
              "(every (b, h) stream is independent; multi-GPU sharding is not part of this build). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    B, T, H, K = args.B, args.T, args.H, args.d
    main_v = args.variant
    from lit_gpt.kdn_ops import _memscan
    if args.serial_schedule:
        _memscan.DEFAULT_OVERLAP = False
    _memscan.set_backward_mode(args.backward_mode)
    if args.decode_only:
        line = run_decode(f"{main_v}_kdn_1.3B", max(args.steps, 20), args.warmup)
        print(json.dumps(dict(line, metric=f"{main_v}_kdn_1.3B decode tokens/s")), flush=True)
        return
    if args.config3_only:
        line = run_config3(args.steps, args.warmup)
        print(json.dumps(dict(line, metric="diag_kdn long-context forward tokens/s (config 3)")), flush=True)
        return
    if args.config4_only:
        line = run_config4(f"{main_v}_kdn_1.3B", args.steps, args.warmup, 1, T)
        print(json.dumps(dict(line, metric=f"{main_v}_kdn_1.3B forward tokens/s (config 4)")), flush=True)
        return
    other = "diag" if main_v == "iso" else "iso"
    res = run_variant(main_v, args.steps, args.warmup, B, T, H, K)
    if args.headline_only:
        if args.calib_copy:
            calib_copy(args.calib_copy)
        print(json.dumps({"metric": METRIC, "value": round(res["tokens_per_s"], 1), "unit": "tokens/s",
                          "ms_per_step": round(res["ms_per_step"], 4), "steps": args.steps, "warmup": args.warmup,
                          "roofline": headline_roofline(main_v, res["dominant"], res["kernels"][res["dominant"]],
                                                        B, T, H, K),
                          "op_roofline": op_roofline(main_v, res["ms_per_step"], B, T, H, K),
                          "kernels": res["kernels"]}), flush=True)
        return
    res_other = run_variant(other, args.steps, args.warmup, B, T, H, K)
    dom = res["kernels"][res["dominant"]]
    cfg_key = f"{main_v} B{B} T{T} H{H} d{K}"
    traffic = measured_traffic(res["dominant"], cfg_key)
    line = {
        "metric": METRIC,
        "value": round(res["tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 inputs / fp32 state",
        "data": "synthetic",
        "config": {"workload": f"{main_v}_kdn mixer scan fwd+bwd (frontend+gain+chunked memory, all input grads)",
                   "B": B, "T": T, "H": H, "d_k": K, "d_v": K, "chunk": C, "inputs": "bf16",
                   "state": "fp32", "parallelism": "single GPU"},
        "roofline": headline_roofline(main_v, res["dominant"], dom, B, T, H, K, traffic),
        "op_roofline": op_roofline(main_v, res["ms_per_step"], B, T, H, K),
        "kernels": res["kernels"],
        "also": {f"{other}_kdn": {"value": round(res_other["tokens_per_s"], 1), "unit": "tokens/s",
                                  "ms_per_step": round(res_other["ms_per_step"], 4),
                                  "op_roofline": op_roofline(other, res_other["ms_per_step"], B, T, H, K),
                                  "roofline": headline_roofline(other, res_other["dominant"],
                                                                res_other["kernels"][res_other["dominant"]], B, T, H,
                                                                K, measured_traffic(res_other["dominant"],
                                                                                    f"{other} B{B} T{T} H{H} d{K}")),
                                  "dominant": res_other["dominant"],
                                  "kernels": res_other["kernels"]},
                 "layer_frontends": {"workload": "packed q|k|v short conv + SiLU and sigmoid-gated RMS norm, "
                                                 "fwd+bwd, bf16, same B/T/H/d",
                                     "kernels": run_layer_frontends(args.steps, args.warmup, B, T, H, K)}},
    }
    if args.backward_mode == "save":
        # the same steps with the reference's memory policy: the forward keeps only the op's inputs and
        # the backward rebuilds the intra-chunk factors and per-chunk states first
        _memscan.set_backward_mode("recompute")
        rec = {v: run_variant(v, min(args.steps, 10), args.warmup, B, T, H, K)["ms_per_step"] for v in ("iso", "diag")}
        _memscan.set_backward_mode("save")
        line["also"]["recompute_backward"] = {
            "ms_per_step": {v: round(x, 4) for v, x in rec.items()},
            "tokens_per_s": {v: round(B * T / (x * 1e-3), 1) for v, x in rec.items()},
            "saved_bytes_save_mode": _lib_size("kdn_mem_saved_size", B, T, H, K, K),
            "note": "forward keeps the op's inputs only (no WY factors, A^T or per-chunk states); identical gradients"}
    if not args.no_config3:
        line["also"]["config3"] = run_config3(min(args.steps, 10), args.warmup)
    if not args.no_config4:
        line["also"]["config4"] = run_config4(f"{main_v}_kdn_1.3B", min(args.steps, 10), args.warmup, 1, T)
    if not args.no_decode:
        line["also"]["decode"] = run_decode(f"{main_v}_kdn_1.3B", max(args.steps, 20), args.warmup)
    if args.calib_copy:
        calib_copy(args.calib_copy)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(main_v, args.cpu_slices, T, K, B, H)
        line["also"][f"{other}_kdn"]["cpu_baseline"] = cpu_baseline(other, args.cpu_slices, T, K, B, H)
        if not args.no_config3:
            line["also"]["config3"]["cpu_baseline"] = cpu_baseline_config3(32768, K, 1, H)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
