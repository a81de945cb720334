"""Token-by-token decoding of a KDN ``GPT`` with the layers' recurrent state kept on the GPU.

The reference has no decoding path for KDN models (``model.py:104,184`` refuse caching).  Every
KDN layer's history is a fixed-size state (``KDNLayerState``), so a decode step costs the same at
any context length: the chunked scan consumes the prompt (``prefill``), then each ``step`` runs
one token through every block, the mixers through ``kdn_kalman_step``.

One decode step launches a few hundred small kernels (about 20 per block), so at small batch
the step is bound by launch overhead, not by the GPU.  With ``use_graph=True`` the step is
captured once as a HIP graph (``torch.cuda.CUDAGraph``) over fixed buffers -- the token ids, the
logits and every layer's state -- and each later step is one graph replay.  The decoder's layer
states are in-place states (``KDNLayerState.inplace``): each layer advances its own buffers, the
mixers through ``kdn_kalman_step`` (the single-token gain and memory update in one launch).
"""
from __future__ import annotations

import torch

from .kdn_state import KDNLayerState


class KDNDecoder:
    def __init__(self, model, batch_size: int, *, use_graph: bool = True):
        self.model = model
        self.B = int(batch_size)
        self.use_graph = bool(use_graph)
        self.state = None
        self.graph = None
        dev = next(model.parameters()).device
        self.tokens = torch.zeros(self.B, 1, dtype=torch.long, device=dev)
        self.logits = None

    @torch.no_grad()
    def prefill(self, idx: torch.Tensor) -> torch.Tensor:
        """Run the prompt ``idx`` [B,T] (T >= 1) through the chunked scan; returns its logits [B,T,V]
        and keeps the state after it (copied into this decoder's fixed buffers)."""
        if idx.ndim != 2 or idx.shape[0] != self.B:
            raise ValueError(f"idx must have shape [{self.B}, T], got {tuple(idx.shape)}")
        logits, state = self.model(idx, return_state=True)
        if self.state is None:
            self.state = [KDNLayerState(tuple(c.clone() for c in s.conv), s.memory.clone(), s.precision.clone(),
                                        s.seen_tokens, inplace=True) for s in state]
            self.logits = torch.empty_like(logits[:, -1])
        else:
            self._assign(state)
            for s, n in zip(self.state, state):
                s.seen_tokens = n.seen_tokens
        return logits

    def _assign(self, new):
        for s, n in zip(self.state, new):
            s.memory.copy_(n.memory)
            s.precision.copy_(n.precision)
            for c, nc in zip(s.conv, n.conv):
                c.copy_(nc)

    def _eager_step(self):
        # the states are in-place states: the layers advance their buffers themselves
        logits, _ = self.model(self.tokens, state=self.state, return_state=True)
        self.logits.copy_(logits[:, -1])

    def _capture(self):
        # warm up (library handles, allocator) on a side stream without advancing the state
        saved = [(s.memory.clone(), s.precision.clone(), tuple(c.clone() for c in s.conv), s.seen_tokens)
                 for s in self.state]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                self._eager_step()
        torch.cuda.current_stream().wait_stream(side)
        for s, (m, p, cs, n) in zip(self.state, saved):
            s.memory.copy_(m)
            s.precision.copy_(p)
            for c, sc in zip(s.conv, cs):
                c.copy_(sc)
            s.seen_tokens = n
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._eager_step()
        for s, (_, _, _, n) in zip(self.state, saved):
            s.seen_tokens = n  # capture records the step without running it

    @torch.no_grad()
    def step(self, tokens: torch.Tensor) -> torch.Tensor:
        """Feed one token per sequence (``tokens`` [B] or [B,1]); returns the next-token logits [B,V]
        (a view of this decoder's buffer, overwritten by the next step)."""
        if self.state is None:
            raise RuntimeError("call prefill() before step()")
        self.tokens.copy_(tokens.view(self.B, 1))
        if not self.use_graph:
            self._eager_step()  # advances seen_tokens itself
        else:
            if self.graph is None:
                self._capture()
            self.graph.replay()
            for s in self.state:
                s.seen_tokens += 1
        return self.logits


__all__ = ("KDNDecoder",)
