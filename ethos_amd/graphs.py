"""Graph-captured forwards of the expert layer for serving loops.

A decode step of the layer is a chain of about ten short kernels (query projection,
routing, sort, generation, activations, scatter-back) whose host-side launch work is
comparable to their GPU time at small batches.  `CapturedLayer` records one forward for a
fixed input shape into a HIP graph (torch.cuda.CUDAGraph) and replays it: per call one
copy of the input into the captured buffer and one graph launch.  Optionally
(`overlap_token_proj`) the token projection x W_u, which needs only x, runs on a second
stream inside the graph beside the query projection, routing and sort, and joins before the
expert stages; on ROCm 7 the fork and join cost more GPU time than the overlap saves (64
tokens: 0.167 against 0.153 ms per replayed step), so it is off by default.

The replay gives the eager forward's output bit for bit (the same kernels on the same
inputs).  The graph holds the layer's packed parameters by address: when a parameter or a
BatchNorm buffer changes (its version counter moves), the next call captures again.
"""
from __future__ import annotations

import torch

from .layer import EthosExpertLayer


class CapturedLayer:
    """One eval-mode forward of `layer` on [n_tok, d_model] rows, captured and replayed.

    `layer(x)` and `captured(x)` give the same output for x of that shape.  The returned
    tensor is the graph's output buffer: the next call overwrites it (clone it to keep it).
    `overlap_token_proj` runs the token projection on a second stream inside the graph.
    Calls on one CapturedLayer must not overlap (one input and one output buffer)."""

    def __init__(self, layer: EthosExpertLayer, n_tok: int, dtype: torch.dtype | None = None,
                 device: torch.device | str | None = None, overlap_token_proj: bool = False, warmup: int = 2):
        if not isinstance(layer, EthosExpertLayer):
            raise TypeError("CapturedLayer wraps an EthosExpertLayer")
        if layer.training or layer.router._bn_uses_batch_stats():
            raise RuntimeError("CapturedLayer needs the layer in eval mode (BatchNorm with running statistics)")
        if n_tok <= 0:
            raise ValueError("n_tok must be positive")
        p = layer.expert_latents.weight
        self.layer = layer
        self.n_tok = int(n_tok)
        self.dtype = dtype or p.dtype
        self.device = torch.device(device) if device is not None else p.device
        if self.device.type != "cuda":
            raise RuntimeError("CapturedLayer needs the layer on a HIP device")
        self.overlap_token_proj = overlap_token_proj
        self.warmup = max(1, int(warmup))
        self.input = torch.zeros((self.n_tok, layer.d_model), dtype=self.dtype, device=self.device)
        self._capture()

    def _state(self):
        # looked up afresh on every call: a parameter replaced by a new object counts as a change
        return tuple((t.data_ptr(), t._version) for t in self.layer._param_sources() if t is not None)

    def _capture(self) -> None:
        layer = self.layer
        self._side = torch.cuda.Stream(device=self.device) if self.overlap_token_proj else None
        side = self._side
        # warm up off the capture (builds the layer's parameter caches) on a side stream, as
        # graph capture asks
        warm = torch.cuda.Stream(device=self.device)
        warm.wait_stream(torch.cuda.current_stream(self.device))
        with torch.no_grad(), torch.cuda.stream(warm):
            for _ in range(self.warmup):
                layer.forward_flat(self.input, side_stream=side)
        torch.cuda.current_stream(self.device).wait_stream(warm)
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(self.graph):
            self.output = layer.forward_flat(self.input, side_stream=side)
        self._key = self._state()

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if x.dim() == 3:
            x = x.reshape(-1, x.shape[-1])
        if x.shape != self.input.shape or x.dtype != self.dtype or x.device != self.input.device:
            raise RuntimeError(f"CapturedLayer takes {tuple(self.input.shape)} {self.dtype} on {self.input.device}, "
                               f"got {tuple(x.shape)} {x.dtype} on {x.device}")
        if self._state() != self._key:
            self._capture()
        self.input.copy_(x)
        self.graph.replay()
        return self.output
