"""ctypes binding of the C ABI in include/kdn.h (libkdn_hip.so, built for gfx950).

Every op in this package calls through here; there is no CPU or PyTorch fallback.
If the library is missing the first call raises RuntimeError.
"""
from __future__ import annotations

import ctypes
import os
import pathlib

import torch

_LIB_PATH = pathlib.Path(__file__).resolve().parent / "libkdn_hip.so"
_lib = None

# Argument codes: p pointer, i int, l int64, f float, z size_t, s hipStream_t
_SIGS = {
    "kdn_iso_gate_fwd": "pipillpppppffiiiiippppps",
    "kdn_iso_gate_bwd_workspace_size": "iiiii",
    "kdn_iso_gate_bwd": "pipillppppppppppiiiiippppppppzs",
    "kdn_iso_gain_workspace_size": "iii",
    "kdn_iso_gain_fwd": "ppppiiiifppppzs",
    "kdn_iso_gain_fwd_noalloc": "ppppiiiifppps",
    "kdn_iso_gain_bwd": "ppppippppiiifpppppzs",
    "kdn_iso_front_workspace_size": "iiii",
    "kdn_iso_front_fwd": "pipill" "ppppp" "ff" "pi" "iiii" "f" "pppppppp" "pzs",
    "kdn_iso_front_bwd": "pipill" "pppppp" "i" "ppppppppp" "iiii" "f" "pppppppp" "pzs",
    "kdn_l2norm_fwd": "pilifpips",
    "kdn_l2norm_bwd": "pippilips",
    "kdn_diag_norm_fwd": "ppilippppps",
    "kdn_diag_norm_bwd": "ppippppplipps",
    "kdn_diag_frontend_fwd": "ppppppiiiiippppps",
    "kdn_diag_frontend_bwd_workspace_size": "iiiii",
    "kdn_diag_frontend_bwd": "ppppppppppppiiiiipppppppzs",
    "kdn_diag_gain_workspace_size": "iiii",
    "kdn_diag_gain_fwd": "pppppiiiiifpppppzs",
    "kdn_diag_gain_bwd": "pppppipppppppiiiifpppppppzs",
    "kdn_diag_front_saved_size": "iiii",
    "kdn_diag_front_workspace_size": "iiii",
    "kdn_diag_front_fwd": "pipppppppp" "iiiiii" "f" "pppppzs",
    "kdn_diag_front_bwd": "pipppppppp" "i" "pppppp" "iiiii" "f" "ppppppppp" "zs",
    "kdn_mem_chunk_size": "",
    "kdn_mem_state_groups": "iiiii",
    "kdn_mem_saved_size": "iiiii",
    "kdn_mem_bwd_workspace_size": "iiiii",
    "kdn_mem_fwd": "pppippiiiiifppzppippis",
    "kdn_mem_bwd": "pppipiiiiifpippzpzpppppppppis",
    "kdn_mem_step": "pppipipiiiifppis",
    "kdn_kalman_step": "pppipppppppiiiiiffppis",
    "kdn_gemv": "pilppiiiipls",
    "kdn_xent_fwd": "pilpiiifffllliippps",
    "kdn_xent_bwd": "plplpilppiiifffllls",
    "kdn_short_conv_fwd": "pillpiiiiiplls",
    "kdn_short_conv_step": "pilplpiiipls",
    "kdn_short_conv_bwd_workspace_size": "iii",
    "kdn_short_conv_bwd": "pillpiplliiiiipllppzs",
    "kdn_rms_norm_fwd": "pipilifpps",
    "kdn_rms_norm_bwd_workspace_size": "li",
    "kdn_rms_norm_bwd": "pipipplipppzs",
    "kdn_rms_norm_gated_fwd": "pipipilifipps",
    "kdn_rms_norm_gated_bwd_workspace_size": "li",
    "kdn_rms_norm_gated_bwd": "pipipippliippppzs",
}
_SIZE_FNS = {"kdn_iso_gate_bwd_workspace_size", "kdn_iso_gain_workspace_size", "kdn_iso_front_workspace_size",
             "kdn_diag_frontend_bwd_workspace_size",
             "kdn_diag_gain_workspace_size", "kdn_diag_front_saved_size",
             "kdn_diag_front_workspace_size", "kdn_mem_saved_size", "kdn_mem_bwd_workspace_size",
             "kdn_short_conv_bwd_workspace_size", "kdn_rms_norm_gated_bwd_workspace_size",
             "kdn_rms_norm_bwd_workspace_size"}
_CT = {"p": ctypes.c_void_p, "i": ctypes.c_int, "l": ctypes.c_int64, "f": ctypes.c_float,
       "z": ctypes.c_size_t, "s": ctypes.c_void_p}


def library_path() -> pathlib.Path:
    return _LIB_PATH


def load():
    """Load libkdn_hip.so (after torch has initialised its HIP runtime) and declare signatures."""
    global _lib
    if _lib is not None:
        return _lib
    if not _LIB_PATH.exists():
        raise RuntimeError(
            f"KDN HIP library not found at {_LIB_PATH}; build it with "
            "`python kalman-delta-networks_amd/build_hip.py` (there is no fallback path)")
    # The library links libamdhip64.so.7; loading torch first makes it bind to torch's runtime.
    lib = ctypes.CDLL(str(_LIB_PATH), mode=os.RTLD_LOCAL)
    for name, sig in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = [_CT[c] for c in sig]
        fn.restype = ctypes.c_size_t if name in _SIZE_FNS else ctypes.c_int
    _lib = lib
    return lib


def exported_symbols() -> tuple[str, ...]:
    return tuple(_SIGS)


def ptr(t):
    """Device pointer of a tensor (or None -> NULL)."""
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


class KernelTimer:
    """Records HIP events on the launching stream around every tagged C call while active.

    Used by the benchmark to time individual kernels inside the timed region."""

    def __init__(self):
        self.events: dict[str, list] = {}

    def __enter__(self):
        global _timer
        _timer = self
        return self

    def __exit__(self, *exc):
        global _timer
        _timer = None
        return False

    def mean_ms(self, tag: str) -> float:
        pairs = self.events.get(tag, [])
        if not pairs:
            return float("nan")
        torch.cuda.synchronize()
        return sum(s.elapsed_time(e) for s, e in pairs) / len(pairs)

    def tags(self):
        return tuple(self.events)


_timer: KernelTimer | None = None


def timing() -> bool:
    """True while a KernelTimer is active (callers then launch one kernel per call)."""
    return _timer is not None


def call(name: str, *args, tag: str | None = None):
    """Call entry point ``name``; under a KernelTimer the call is timed as ``tag`` (default: the
    entry name without its ``kdn_`` prefix)."""
    lib = load()
    fn = getattr(lib, name)
    if _timer is not None:
        if tag is None:
            tag = name[4:] if name.startswith("kdn_") else name
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        rc = fn(*args)
        end.record()
        _timer.events.setdefault(tag, []).append((start, end))
    else:
        rc = fn(*args)
    if rc != 0:
        raise RuntimeError(f"{name} failed with code {rc}"
                           + (" (invalid argument)" if rc == -1 else " (HIP error)"))


def size(name: str, *args) -> int:
    return int(getattr(load(), name)(*args))


def is_bf16(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return 1
    if t.dtype == torch.float32:
        return 0
    raise TypeError(f"expected bf16 or fp32 tensor, got {t.dtype}")


def require_device(*tensors):
    """All tensors must live on one ROCm device; the HIP library runs nowhere else."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("KDN HIP ops require tensors on a ROCm (cuda) device")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all KDN tensors must share one device")
    return dev
