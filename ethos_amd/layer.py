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
tensors; there is no CPU path.

With autograd enabled (the input or a parameter requires grad, outside torch.no_grad)
the output carries a graph whose gradients are those of the reference's pure-PyTorch
layer (model.py:288-343, differentiated by autograd there): through the routing gates
to the query projections, BatchNorm affine parameters and sub-keys (the topk values
and softmax, model.py:215-234), and through the generated experts to x, the expert
latents and both generator weights.  The forward values are the HIP kernels' in both
cases; the reference's Triton layer (kernels.py:145-221) has no backward at all.
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


def _gelu_grad(x: torch.Tensor) -> torch.Tensor:
    """Derivative of the erf GELU x·Φ(x): Φ(x) + x·φ(x)."""
    cdf = 0.5 * (1.0 + torch.erf(x * (1.0 / math.sqrt(2.0))))
    pdf = torch.exp(-0.5 * x * x) * (1.0 / math.sqrt(2.0 * math.pi))
    return cdf + x * pdf


class _ExpertStages(torch.autograd.Function):
    """Expert generation, apply and scatter-back as one autograd node.

    Forward: the HIP generator and apply kernels, given the routing (gates, the sorted
    pair segments).  Backward: the derivative of the reference's per-pair expression
    (model.py:312-341), evaluated in float32 from the saved routing and generated rows.
    With A = W2[:d], B = W2[d:] (net.2.weight halves), C = W1 (net.0.weight), pair p of
    token t(p) using unique expert s(p):

        pre_s = z_s C^T,  h_s = gelu(pre_s),  v_s = h_s B^T,  xp_t = x_t A,
        c_p = h_s · xp_t,  a_p = gelu(c_p) g_p,  y_t = (1/H) Σ_p a_p v_s

    so with dY_t = dy_t / H:  da_p = dY_t · v_s = (dY_t B) · h_s;  dg_p = gelu(c_p) da_p;
    dc_p = g_p gelu'(c_p) da_p;  dxp_t = Σ_p dc_p h_s;  dh_s = Σ_p (dc_p xp_t + a_p dY_t B);
    dA = x^T dxp,  dB = dY^T hacc with hacc_t = Σ_p a_p h_s,  dx = dxp A^T;
    dpre = gelu'(pre) dh,  dC = dpre^T z,  dz = dpre C (added into the latent rows of the
    unique experts).  v rows are not needed.  The per-pair terms, the token sums (hacc, dxp)
    and the expert sums (dh, summed over each expert's sorted pairs in a fixed order) come
    from one library call (ethos_expert_backward); the rest are GEMMs.  The backward is
    deterministic.  Both execution orders (scatter of v rows, hidden-space reordering)
    compute this same function, so they share the backward.

    The gates enter as `gates_exact` (the values the forward uses) and `gate_path` (a
    float32 tensor of the same values carrying the router's graph), whose gradient is dg.
    """

    @staticmethod
    def forward(ctx, x, gate_path, latents_w, w1_w, w2_w, layer, gates_exact, seg):
        out, h = layer._expert_stages(x, gates_exact, seg)
        latents, w1, w2, _ = layer._generator_params(x.dtype, x.device)
        ctx.save_for_backward(x, gates_exact, h, seg["uniq"], seg["pair_slot"], seg["n_unique"], seg["perm"],
                              seg["sorted_slot"], seg["seg_off"], latents, w1, w2)
        ctx.heads, ctx.top_k = layer.num_heads, layer.top_k
        ctx.param_dtypes = (latents_w.dtype, w1_w.dtype, w2_w.dtype)
        return out

    @staticmethod
    def backward(ctx, dy):
        # v_s = h_s B^T never needs forming: dY_t . v_s = (dY_t B) . h_s, the dv_s B term of
        # dh_s is sum_p a_p (dY_t B), and dB = dv^T h = dY^T hacc with hacc_t = sum_p a_p h_s.
        x, gates, h, uniq, pair_slot, n_unique, perm, sorted_slot, seg_off, latents, w1, w2 = ctx.saved_tensors
        seg = {"pair_slot": pair_slot, "perm": perm, "sorted_slot": sorted_slot, "seg_off": seg_off}
        H, k = ctx.heads, ctx.top_k
        n, d = x.shape
        f = torch.float32
        U = int(n_unique.item())
        A, B, C = w2[:d].to(f), w2[d:].to(f), w1.to(f)
        xf = x.to(f)
        xp = xf @ A
        dY = dy.to(f) * (1.0 / H)
        dYB = dY @ B
        # per-pair terms, token sums and expert sums (ethos_expert_backward)
        dg, hacc, dxp, dh = hip.expert_backward(h, xp, dYB, seg, gates, H, k, U)
        dB = dY.T @ hacc
        dA = xf.T @ dxp
        dx = dxp @ A.T
        ids = uniq[:U].long()
        z = latents[ids].to(f)
        dpre = _gelu_grad(z @ C.T) * dh
        dC = dpre.T @ z
        dlat = torch.zeros(latents.shape, dtype=f, device=x.device)
        dlat.index_add_(0, ids, dpre @ C)
        lat_dt, w1_dt, w2_dt = ctx.param_dtypes
        return (dx.to(x.dtype), dg.view(gates.shape), dlat.to(lat_dt), dC.to(w1_dt),
                torch.cat([dA, dB], 0).to(w2_dt), None, None, None)


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
        self._keys_prepared = None
        self._wq_prepared = None

    # -- parameter packing (cached until a parameter changes) ---------------------
    def _packed_sources(self) -> list:
        """The tensors the packed form is built from, read from the modules' parameter and
        buffer dicts directly (this runs on every call; nn.Module attribute lookup is slow)."""
        ts = []
        for m in self._modules["query_projs"]._modules.values():
            ts += (m._parameters["weight"], m._parameters["bias"])
        ts += (self._modules["sub_keys_1"]._parameters["weight"], self._modules["sub_keys_2"]._parameters["weight"])
        for m in self._modules["query_norms"]._modules.values():
            ts += (m._parameters["weight"], m._parameters["bias"], m._buffers["running_mean"], m._buffers["running_var"])
        return ts

    def _packed(self, dtype: torch.dtype, device: torch.device):
        key = (dtype, device, tuple((t.data_ptr(), t._version) for t in self._packed_sources() if t is not None))
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
            # the sub-keys in the scoring MFMAs' fragment order
            self._keys_prepared = hip.route_prepare_keys(k1, k2) if k1.is_cuda else None
            # the projection weights' prepared form (bf16: digit planes), reused by every call
            # until a parameter changes
            self._wq_prepared = hip.query_proj_prepare(wq) if wq.is_cuda else None
            self._cache = (wq, bq, k1, k2, alpha, beta)
            self._cache_key = key
        return self._cache

    def _bn_uses_batch_stats(self) -> bool:
        return any(m.training or not m.track_running_stats for m in self.query_norms)

    def queries(self, x_flat: torch.Tensor, packed=None) -> torch.Tensor:
        """Per-head queries after BatchNorm, [n, H, d_query] (model.py:215-216).  `packed`:
        the result of _packed for x_flat's dtype and device, if the caller has it."""
        wq, bq, _, _, alpha, beta = packed if packed is not None else self._packed(x_flat.dtype, x_flat.device)
        if not self._bn_uses_batch_stats():
            return hip.query_proj(x_flat, wq, bq, alpha, beta, prepared=self._wq_prepared)
        # Training-mode BatchNorm normalises with batch statistics and updates the
        # running stats: project with an identity affine, then apply torch's batch_norm
        # per head on the projected queries.
        ones = torch.ones_like(alpha)
        zeros = torch.zeros_like(beta)
        q_lin = hip.query_proj(x_flat, wq, bq, ones, zeros, prepared=self._wq_prepared)
        outs = []
        for h, m in enumerate(self.query_norms):
            outs.append(F.batch_norm(q_lin[:, h], m.running_mean, m.running_var,
                                     m.weight if m.affine else None, m.bias if m.affine else None,
                                     m.training or not m.track_running_stats, m.momentum if m.momentum is not None else 0.1,
                                     m.eps))
            if m.training and m.track_running_stats:
                m.num_batches_tracked.add_(1)
        # batch_norm updated the running statistics in place without bumping their version
        # counters, so the eval-mode coefficients cached by _packed are stale
        if any(m.training and m.track_running_stats for m in self.query_norms):
            self._cache_key = None
        return torch.stack(outs, dim=1).contiguous()

    def route(self, x_flat: torch.Tensor, mark=None):
        """(gates [n, H, k] x.dtype, expert ids [n, H, k] int32).  `mark(stage)`, if given,
        is called after each stage is enqueued (used to place timing events)."""
        packed = self._packed(x_flat.dtype, x_flat.device)
        _, _, k1, k2, _, _ = packed
        q = self.queries(x_flat, packed)
        if mark is not None:
            mark("query_proj")
        out = hip.route_topk(q, k1, k2, self.top_k, key_norms=self._key_norms, prepared_keys=self._keys_prepared)
        if mark is not None:
            mark("route")
        return out

    def gate_path(self, x_flat: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
        """float32 gates [n, H, k] recomputed with torch operations from the chosen expert ids,
        carrying autograd to x, the query projections, the BatchNorm affine parameters and
        both sub-key tables as the reference's topk values and softmax do (model.py:215-234):
        g = softmax(q1 · K1[i1] + q2 · K2[i2]) with i1 = id // K, i2 = id % K.  BatchNorm uses
        the module's mode (batch statistics when training) without touching the running
        statistics, which the routing pass has already updated."""
        f = torch.float32
        H, dq, K = self.num_heads, self.d_query, self.num_sub_keys
        n = x_flat.shape[0]
        w = torch.stack([m.weight for m in self.query_projs]).to(f).reshape(H * dq, -1)
        b = torch.stack([m.bias for m in self.query_projs]).to(f).reshape(-1)
        q = x_flat.to(f) @ w.T + b                                       # [n, H dq]
        # the H per-head BatchNorms as one over H dq channels (same per-channel statistics)
        norms = list(self.query_norms)
        batch = [m.training or not m.track_running_stats for m in norms]
        if all(batch) or not any(batch):
            cat = lambda ts: torch.cat([t.to(f) for t in ts])  # noqa: E731
            affine = all(m.affine for m in norms)
            q = F.batch_norm(q, None if batch[0] else cat(m.running_mean for m in norms),
                             None if batch[0] else cat(m.running_var for m in norms),
                             cat(m.weight for m in norms) if affine else None,
                             cat(m.bias for m in norms) if affine else None,
                             batch[0], 0.0, norms[0].eps) if len({m.eps for m in norms}) == 1 else None
        else:
            q = None
        if q is None:  # heads in different modes or with different eps: one call per head
            q = (x_flat.to(f) @ w.T + b).view(n, H, dq)
            q = torch.stack([F.batch_norm(q[:, h], None if bt else m.running_mean.to(f),
                                          None if bt else m.running_var.to(f),
                                          m.weight.to(f) if m.affine else None, m.bias.to(f) if m.affine else None,
                                          bt, 0.0, m.eps) for h, (m, bt) in enumerate(zip(norms, batch))], dim=1)
        q = q.view(n * H, dq)
        half = dq // 2
        # dense sub-scores, then the chosen columns: the backward is a GEMM for the keys
        s1 = (q[:, :half] @ self.sub_keys_1.weight.to(f).T).gather(1, (ids // K).view(n * H, -1))
        s2 = (q[:, half:] @ self.sub_keys_2.weight.to(f).T).gather(1, (ids % K).view(n * H, -1))
        return torch.softmax(s1 + s2, dim=-1).view(ids.shape)

    def forward(self, x_flat: torch.Tensor):
        """(scores [n, H, k], expert ids [n, H, k] int64) as model.py:208-254.  With autograd
        enabled the scores carry the gradient of the reference's topk + softmax."""
        with torch.no_grad():
            gates, ids = self.route(_as_input(x_flat, 2))
        ids = ids.long()
        if _wants_grad(x_flat, self):
            g = self.gate_path(x_flat, ids)
            gates = gates + (g - g.detach()).to(gates.dtype)
        return gates, ids


class EthosExpertLayer(nn.Module):
    """The ETHOS expert layer: product-key routing over num_experts generated experts,
    reordered execution by expert id, head-averaged weighted scatter-back."""

    def __init__(self, config, hidden_space: bool | None = None):
        super().__init__()
        self.d_model = config.d_model
        self.num_experts = config.num_experts
        self.top_k = config.top_k
        self.num_heads = config.num_routing_heads
        self.d_latent = config.d_latent
        self.d_hidden = config.d_intermediate_hypernet
        # Execution order of the expert stages: False (default) generates v_e = h_e W_v per
        # unique expert and scatters a_p v_e into the tokens (model.py:320-341, the layer's
        # rounding points); True is the paper's hidden-space reordering (Algorithm 1,
        # paper/ETHOS.pdf p.10): h_acc = sum_p a_p h_e per token, projected by W_v once.
        # Same function, different rounding points; no v rows.
        self.hidden_space = bool(getattr(config, "hidden_space", False) if hidden_space is None else hidden_space)
        self.expert_latents = nn.Embedding(config.num_experts, config.d_latent)
        self.generation_network = ExpertGenerationNetwork(config.d_latent, config.d_model,
                                                          config.d_intermediate_hypernet)
        self.router = ProductKeyRouter(config)
        self._gen_key = None
        self._gen = None

    def _param_sources(self) -> list:
        """Every tensor a forward reads (router parameters and BatchNorm buffers, latents and
        both generator weights), looked up afresh through the modules' dicts, so that a
        replaced parameter object is seen too."""
        gen = self._modules["generation_network"]._modules["net"]._modules
        return self._modules["router"]._packed_sources() + [
            self._modules["expert_latents"]._parameters["weight"], gen["0"]._parameters["weight"],
            gen["2"]._parameters["weight"]]

    def _generator_params(self, dtype, device):
        """(latents, W1, W2, W_u^T): the generator weights in the layer dtype on the device,
        and (bf16) the transpose of W2's first d_model rows, cached until a weight changes."""
        ps = (self.expert_latents.weight, self.generation_network.net[0].weight, self.generation_network.net[2].weight)
        key = (dtype, device, tuple((p.data_ptr(), p._version) for p in ps))
        if key != self._gen_key:
            if all(p.dtype == dtype and p.device == device and p.is_contiguous() for p in ps):
                gen = tuple(p.detach() for p in ps)
            else:
                gen = tuple(p.detach().to(device=device, dtype=dtype).contiguous() for p in ps)
            wut = gen[2][: self.d_model].t().contiguous() if dtype == torch.bfloat16 else None
            self._gen = gen + (wut,)
            self._gen_key = key
        return self._gen

    def _expert_stages(self, x_flat: torch.Tensor, gates: torch.Tensor, seg: dict, xp: torch.Tensor | None = None):
        """(out, h): generation over the unique experts, activations and scatter-back in the
        layer's execution order, as one library call (`xp`: the token projection, if already
        formed)."""
        latents, w1, w2, wut = self._generator_params(x_flat.dtype, x_flat.device)
        return hip.expert_forward(x_flat, latents, w1, w2, seg, gates, self.num_heads, self.top_k,
                                  hidden_space=self.hidden_space, wut=wut, xp=xp)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dim() != 3 or x.shape[-1] != self.d_model:
            raise RuntimeError(f"expected x of shape [batch, seq, {self.d_model}], got {tuple(x.shape)}")
        b, s, d = x.shape
        x_flat = _as_input(x, 3).view(-1, d)
        if x_flat.shape[0] == 0:
            return torch.zeros_like(x)
        return self.forward_flat(x_flat).view(b, s, d)

    def forward_flat(self, x_flat: torch.Tensor, mark=None, side_stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """The layer on [n_tok, d_model] rows (model.py:288-343).  `mark(stage)`, if given, is
        called after the query projection, the routing and the sort are enqueued on the
        current stream (the expert stages are one library call; hip.stage_events times the
        stages inside it).  `side_stream`: the token projection x W_u, which needs only x, runs
        there while the routing and the sort run on the current stream, which waits for it
        before the expert stages (worth its host cost under graph capture; see
        ethos_amd.graphs)."""
        if _wants_grad(x_flat, self):
            with torch.no_grad():
                gates, ids = self.router.route(x_flat)
                seg = hip.sort_segment(ids.view(-1), self.num_experts)
            g = self.router.gate_path(x_flat, ids.long())
            return _ExpertStages.apply(x_flat, g, self.expert_latents.weight, self.generation_network.net[0].weight,
                                       self.generation_network.net[2].weight, self, gates, seg)
        with torch.no_grad():
            xp = None
            if side_stream is not None:
                cur = torch.cuda.current_stream(x_flat.device)
                _, _, w2, wut = self._generator_params(x_flat.dtype, x_flat.device)
                # allocated on the current stream, written on the side stream, which the
                # current stream waits for before any use
                xp = torch.empty((x_flat.shape[0], self.d_hidden), dtype=x_flat.dtype, device=x_flat.device)
                side_stream.wait_stream(cur)
                with torch.cuda.stream(side_stream):
                    hip.token_proj(x_flat, w2, wut, out=xp)
            gates, ids = self.router.route(x_flat, mark)
            if xp is None and ids.numel() <= hip.SMALL_SORT_MAX and x_flat.dtype == torch.bfloat16:
                # small batches: the token projection runs in the sort's launch, beside its
                # single workgroup
                _, _, w2, wut = self._generator_params(x_flat.dtype, x_flat.device)
                seg, xp = hip.sort_segment_token_proj(ids.view(-1), self.num_experts, x_flat, w2, wut)
            else:
                seg = hip.sort_segment(ids.view(-1), self.num_experts)
            if mark is not None:
                mark("sort_segment")
            if side_stream is not None:
                cur.wait_stream(side_stream)
            out, _ = self._expert_stages(x_flat, gates, seg, xp=xp)
        return out


def _wants_grad(x: torch.Tensor, module: nn.Module) -> bool:
    return torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in module.parameters()))


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
