"""Drop-in ETHOS expert layer for MI355X.

The module tree, constructor, state_dict keys and forward signatures are those of
the reference (wrmedford/ETHOS):

  ExpertGenerationNetwork(d_latent, d_model, d_intermediate)    model.py:168-179
  ProductKeyRouter(config).forward(x_flat) -> (scores, indices)  model.py:182-254
  SimplifiedHypernetMoE(config).forward(x) -> y                  model.py:267-343
  FusedLowRankMoE_Reordered(config).forward(x) -> y              kernels.py:123-221

so ``from ethos_amd import FusedLowRankMoE_Reordered`` replaces the reference import
at model.py:352 and a reference state_dict loads unchanged.  The constructor reads
config.d_model, num_experts (a perfect square), top_k, num_routing_heads, d_latent,
d_intermediate_hypernet and d_query.

Forward runs five HIP stages on the current stream (include/ethos_hip.h): query
projection + BatchNorm, product-key routing, reordering by expert id, expert
generation over the unique experts, and apply + scatter-back.  Inputs must be HIP
tensors; there is no CPU path.  Like the reference Triton layer (kernels.py:145-221),
the forward is not differentiable: the output carries no autograd graph.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import hip


def _bn_eval_coefficients(m: nn.BatchNorm1d, n: int):
    """fp32 coefficients of eval-mode BatchNorm, y = alpha * q + beta (model.py:200-202,216):
    alpha = fp32(w / sqrt(var + eps)), beta = fp32(b - mean * alpha), each evaluated in
    fp64 from the fp32 parameters and rounded once, so the result does not depend on
    which library performs the arithmetic."""
    f64 = lambda t: t.detach().float().cpu().numpy().astype(np.float64)  # noqa: E731
    w = f64(m.weight) if m.affine else np.ones(n)
    b = f64(m.bias) if m.affine else np.zeros(n)
    if m.track_running_stats and m.running_mean is not None:
        mu, var = f64(m.running_mean), f64(m.running_var)
    else:
        mu, var = np.zeros(n), np.ones(n)
    alpha = (w / np.sqrt(var + float(m.eps))).astype(np.float32)
    beta = (b - mu * alpha.astype(np.float64)).astype(np.float32)
    return alpha, beta


class ExpertGenerationNetwork(nn.Module):
    """latent [d_latent] -> [u ; v] [2 d_model] through Linear, GELU, Linear (no biases)."""

    def __init__(self, d_latent: int, d_model: int, d_intermediate: int):
        super().__init__()
        self.d_expert_params = 2 * d_model
        self.net = nn.Sequential(
            nn.Linear(d_latent, d_intermediate, bias=False),
            nn.GELU(),
            nn.Linear(d_intermediate, self.d_expert_params, bias=False),
        )

    def forward(self, latent_vector: torch.Tensor) -> torch.Tensor:
        return self.net(latent_vector)


class ProductKeyRouter(nn.Module):
    """Multi-head product-key router with per-head query BatchNorm and shared sub-keys."""

    def __init__(self, config):
        super().__init__()
        self.d_model = config.d_model
        self.num_experts = config.num_experts
        self.top_k = config.top_k
        self.d_query = config.d_query
        self.num_heads = config.num_routing_heads
        self.num_sub_keys = math.isqrt(self.num_experts)
        if self.num_sub_keys ** 2 != self.num_experts:
            raise AssertionError("num_experts must be a perfect square")
        self.query_projs = nn.ModuleList([nn.Linear(self.d_model, self.d_query) for _ in range(self.num_heads)])
        self.query_norms = nn.ModuleList([nn.BatchNorm1d(self.d_query) for _ in range(self.num_heads)])
        self.sub_keys_1 = nn.Embedding(self.num_sub_keys, self.d_query // 2)
        self.sub_keys_2 = nn.Embedding(self.num_sub_keys, self.d_query // 2)
        self._cache_key = None
        self._cache = None
        self._key_norms = None

    # -- parameter packing (cached until a parameter changes) ---------------------
    def _packed(self, dtype: torch.dtype, device: torch.device):
        params = [p for m in self.query_projs for p in (m.weight, m.bias)]
        params += [self.sub_keys_1.weight, self.sub_keys_2.weight]
        bn = [t for m in self.query_norms for t in (m.weight, m.bias, m.running_mean, m.running_var)]
        key = (dtype, device, tuple((t.data_ptr(), t._version) for t in params + bn))
        if key != self._cache_key:
            wq = torch.stack([m.weight.detach() for m in self.query_projs]).to(device=device, dtype=dtype).contiguous()
            bq = torch.stack([m.bias.detach() for m in self.query_projs]).to(device=device, dtype=dtype).contiguous()
            k1 = self.sub_keys_1.weight.detach().to(device=device, dtype=dtype).contiguous()
            k2 = self.sub_keys_2.weight.detach().to(device=device, dtype=dtype).contiguous()
            alpha, beta = [], []
            for m in self.query_norms:
                a, b = _bn_eval_coefficients(m, self.d_query)
                alpha.append(a)
                beta.append(b)
            alpha = torch.from_numpy(np.stack(alpha)).contiguous().to(device)
            beta = torch.from_numpy(np.stack(beta)).contiguous().to(device)
            self._key_norms = hip.key_norm_bounds(k1, k2).to(device)
            self._cache = (wq, bq, k1, k2, alpha, beta)
            self._cache_key = key
        return self._cache

    def _bn_uses_batch_stats(self) -> bool:
        return any(m.training or not m.track_running_stats for m in self.query_norms)

    def queries(self, x_flat: torch.Tensor) -> torch.Tensor:
        """Per-head queries after BatchNorm, [n, H, d_query] (model.py:215-216)."""
        wq, bq, _, _, alpha, beta = self._packed(x_flat.dtype, x_flat.device)
        if not self._bn_uses_batch_stats():
            return hip.query_proj(x_flat, wq, bq, alpha, beta)
        # Training-mode BatchNorm normalises with batch statistics and updates the
        # running stats: project with an identity affine, then apply torch's batch_norm
        # per head on the projected queries.
        ones = torch.ones_like(alpha)
        zeros = torch.zeros_like(beta)
        q_lin = hip.query_proj(x_flat, wq, bq, ones, zeros)
        outs = []
        for h, m in enumerate(self.query_norms):
            outs.append(F.batch_norm(q_lin[:, h], m.running_mean, m.running_var,
                                     m.weight if m.affine else None, m.bias if m.affine else None,
                                     m.training or not m.track_running_stats, m.momentum if m.momentum is not None else 0.1,
                                     m.eps))
            if m.training and m.track_running_stats:
                m.num_batches_tracked.add_(1)
        return torch.stack(outs, dim=1).contiguous()

    def route(self, x_flat: torch.Tensor, mark=None):
        """(gates [n, H, k] x.dtype, expert ids [n, H, k] int32).  `mark(stage)`, if given,
        is called after each stage is enqueued (used to place timing events)."""
        _, _, k1, k2, _, _ = self._packed(x_flat.dtype, x_flat.device)
        q = self.queries(x_flat)
        if mark is not None:
            mark("query_proj")
        out = hip.route_topk(q, k1, k2, self.top_k, key_norms=self._key_norms)
        if mark is not None:
            mark("route")
        return out

    def forward(self, x_flat: torch.Tensor):
        with torch.no_grad():
            gates, ids = self.route(_as_input(x_flat, 2))
        return gates, ids.long()


class EthosExpertLayer(nn.Module):
    """The ETHOS expert layer: product-key routing over num_experts generated experts,
    reordered execution by expert id, head-averaged weighted scatter-back."""

    def __init__(self, config):
        super().__init__()
        self.d_model = config.d_model
        self.num_experts = config.num_experts
        self.top_k = config.top_k
        self.num_heads = config.num_routing_heads
        self.d_latent = config.d_latent
        self.d_hidden = config.d_intermediate_hypernet
        self.expert_latents = nn.Embedding(config.num_experts, config.d_latent)
        self.generation_network = ExpertGenerationNetwork(config.d_latent, config.d_model,
                                                          config.d_intermediate_hypernet)
        self.router = ProductKeyRouter(config)
        self._gen_key = None
        self._gen = None

    def _generator_params(self, dtype, device):
        ps = (self.expert_latents.weight, self.generation_network.net[0].weight, self.generation_network.net[2].weight)
        key = (dtype, device, tuple((p.data_ptr(), p._version) for p in ps))
        if key != self._gen_key:
            if all(p.dtype == dtype and p.device == device and p.is_contiguous() for p in ps):
                self._gen = tuple(p.detach() for p in ps)
            else:
                self._gen = tuple(p.detach().to(device=device, dtype=dtype).contiguous() for p in ps)
            self._gen_key = key
        return self._gen

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dim() != 3 or x.shape[-1] != self.d_model:
            raise RuntimeError(f"expected x of shape [batch, seq, {self.d_model}], got {tuple(x.shape)}")
        b, s, d = x.shape
        x_flat = _as_input(x, 3).view(-1, d)
        if x_flat.shape[0] == 0:
            return torch.zeros_like(x)
        return self.forward_flat(x_flat).view(b, s, d)

    def forward_flat(self, x_flat: torch.Tensor, mark=None) -> torch.Tensor:
        """The layer on [n_tok, d_model] rows (model.py:288-343).  `mark(stage)`, if given, is
        called after each of the five stages is enqueued on the current stream."""
        with torch.no_grad():
            gates, ids = self.router.route(x_flat, mark)
            seg = hip.sort_segment(ids.view(-1), self.num_experts)
            if mark is not None:
                mark("sort_segment")
            latents, w1, w2 = self._generator_params(x_flat.dtype, x_flat.device)
            h, v = hip.generate(latents, seg["uniq"], seg["n_unique"], seg["max_unique"], w1, w2)
            if mark is not None:
                mark("generate")
            out = hip.apply_scatter(x_flat, w2, h, v, seg, gates, self.num_heads, self.top_k)
            if mark is not None:
                mark("apply_scatter")
        return out


def _as_input(x: torch.Tensor, dim: int) -> torch.Tensor:
    if x.dim() != dim:
        raise RuntimeError(f"expected a {dim}-d input, got shape {tuple(x.shape)}")
    if x.device.type != "cuda":
        raise RuntimeError(f"ETHOS expert layer runs on a HIP device only (input is on {x.device})")
    if not x.is_contiguous():
        # the reference's x.view(-1, d_model) (model.py:290) also requires a viewable input
        raise RuntimeError("input must be contiguous")
    return x


# The reference's two interchangeable layer classes (model.py:351-355).
SimplifiedHypernetMoE = EthosExpertLayer
FusedLowRankMoE_Reordered = EthosExpertLayer
