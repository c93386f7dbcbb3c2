"""The ETHOS language model around the drop-in expert layer (the whole-model forward).

What is shared with the reference's CompressedMoEModel (model.py:367-396) is the interface
only: the module names and parameter shapes of the state_dict (so a reference checkpoint
loads with strict=True), the tied embedding/head, and the function each block computes:
pre-norm multi-head latent attention (model.py:79-165) plus, per block, the expert layer
or, for the first num_dense_layers blocks, a SwiGLU FFN (model.py:257-265).

How it is computed here:
  - the two projections that read the block input (q_a_proj and kv_a_proj_with_mqa) run
    as one GEMM over their stacked weights;
  - the rotary embedding is a rotation of the two halves of each rotary slice by
    per-position angles, applied once to the single rotary key that all heads share
    (model.py:118-125 broadcast it to the heads after rotating);
  - queries, keys and values are written into token-major [batch, seq, heads, width]
    buffers, which SDPA reads through transposed views; the values sit in a buffer as
    wide as the query/key heads (zero columns beyond v_head_dim), the layout the fused
    SDPA kernels take;
  - the dense FFN's gate and up projections run as one GEMM.
The expert layer is EthosExpertLayer (HIP kernels).  Inputs live on a HIP device.
"""
from __future__ import annotations

import math
from types import SimpleNamespace

import torch
import torch.nn as nn
import torch.nn.functional as F

from .layer import EthosExpertLayer

# the reference's configs/default.yaml, with the benchmarked expert-layer shape (d_query
# 256) and the 12-block, all-expert-layer depth of the whole-model workload
LM_DEFAULTS = dict(vocab_size=100277, d_model=1024, num_layers=12, num_heads=16, num_dense_layers=0,
                   q_lora_rank=768, kv_lora_rank=256, v_head_dim=64, qk_nope_head_dim=64, qk_rope_head_dim=64,
                   num_experts=262144, d_latent=128, d_intermediate_hypernet=512, top_k=16, num_routing_heads=8,
                   d_query=256, d_ffn_intermediate=4096, max_seq_len=4096, rms_norm_eps=1e-6, rope_theta=10000.0)


def lm_config(**overrides) -> SimpleNamespace:
    cfg = dict(LM_DEFAULTS)
    cfg.update(overrides)
    return SimpleNamespace(**cfg)


def _stacked(owner: nn.Module, mods) -> torch.Tensor:
    """The weights of several nn.Linear modules stacked along the output dimension.
    Cached on `owner` while no gradient is wanted (until a weight changes); under
    autograd it is rebuilt each call, so gradients reach every weight."""
    ws = [m.weight for m in mods]
    if torch.is_grad_enabled() and any(w.requires_grad for w in ws):
        return torch.cat(ws, 0)
    key = tuple((w.data_ptr(), w._version, w.dtype, w.device) for w in ws)
    if getattr(owner, "_stack_key", None) != key:
        owner._stack = torch.cat([w.detach() for w in ws], 0)
        owner._stack_key = key
    return owner._stack


class RMSNorm(nn.Module):
    """Root-mean-square normalisation with a learned gain: statistics in float32, the
    normalised value rounded to the input dtype, then scaled (model.py:19-30)."""

    def __init__(self, size: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(size))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = F.rms_norm(x.float(), (x.shape[-1],), eps=self.eps)
        return self.weight * y.to(x.dtype)


class Rotary(nn.Module):
    """Rotary position embedding by half-rotation: a slice r = [a, b] of even width 2m at
    position p becomes [a cos t - b sin t, b cos t + a sin t] with t_i = p base^(-2i/2m),
    i < m (model.py:33-76 writes the same rotation with duplicated tables).  Angles,
    cosines and sines are float32, rounded to the activation dtype when used; they are
    formed for the given positions (no table, so no position can fall outside one)."""

    def __init__(self, width: int, base: float):
        super().__init__()
        self.half = width // 2
        self.base = float(base)
        self._rate = None

    def rotate(self, r: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """r [batch, seq, ..., 2m], positions [seq] -> the rotated slice, same shape and dtype."""
        if self._rate is None or self._rate.device != r.device:
            # rates base^(-2i/2m) as the reciprocal of the power, the reference's float32
            # rounding of the frequencies (model.py:40)
            self._rate = 1.0 / self.base ** (torch.arange(0, 2 * self.half, 2, device=r.device,
                                                          dtype=torch.float32) / (2 * self.half))
        ang = positions.to(device=r.device, dtype=torch.float32)[:, None] * self._rate[None, :]
        shape = (1, positions.numel()) + (1,) * (r.dim() - 3) + (self.half,)
        c = ang.cos().to(r.dtype).view(shape)
        s = ang.sin().to(r.dtype).view(shape)
        a, b = r[..., : self.half], r[..., self.half:]
        return torch.cat((a * c - b * s, b * c + a * s), dim=-1)


class MLAttention(nn.Module):
    """Multi-head latent attention.  Queries come from a low-rank bottleneck with an
    RMSNorm; keys and values from a normalised compressed latent, plus one rotary key
    shared by all heads.  Causal softmax attention with scale 1/sqrt(query head width)."""

    def __init__(self, config):
        super().__init__()
        d, H = config.d_model, config.num_heads
        self.n_heads = H
        self.nope, self.rope, self.vdim = config.qk_nope_head_dim, config.qk_rope_head_dim, config.v_head_dim
        self.qk_width = self.nope + self.rope
        self.q_rank, self.kv_rank = config.q_lora_rank, config.kv_lora_rank
        # parameter names and shapes are the checkpoint format (model.py:93-100)
        self.q_a_proj = nn.Linear(d, self.q_rank, bias=False)
        self.q_a_layernorm = RMSNorm(self.q_rank, eps=config.rms_norm_eps)
        self.q_b_proj = nn.Linear(self.q_rank, H * self.qk_width, bias=False)
        self.kv_a_proj_with_mqa = nn.Linear(d, self.kv_rank + self.rope, bias=False)
        self.kv_a_layernorm = RMSNorm(self.kv_rank, eps=config.rms_norm_eps)
        self.kv_b_proj = nn.Linear(self.kv_rank, H * (self.nope + self.vdim), bias=False)
        self.o_proj = nn.Linear(H * self.vdim, d, bias=False)
        self.rotary = Rotary(self.rope, config.rope_theta)
        self.scale = 1.0 / math.sqrt(self.qk_width)

    def forward(self, x: torch.Tensor, attention_mask, position_ids: torch.Tensor) -> torch.Tensor:
        """x [b, n, d].  `attention_mask`: None for causal attention, else an additive
        [n, n] mask (the reference passes triu(-inf, 1), model.py:388-389: the causal
        case).  `position_ids` [n] or [1, n]."""
        b, n, _ = x.shape
        H, nope, rope, w = self.n_heads, self.nope, self.rope, self.qk_width
        pos = position_ids.reshape(-1)
        # one GEMM for both projections of the block input: [q latent | kv latent | rotary key]
        a = F.linear(x, _stacked(self, (self.q_a_proj, self.kv_a_proj_with_mqa)))
        q_lat, kv_lat, k_rot = a.split((self.q_rank, self.kv_rank, rope), dim=-1)
        q = self.q_b_proj(self.q_a_layernorm(q_lat)).view(b, n, H, w)
        kv = self.kv_b_proj(self.kv_a_layernorm(kv_lat)).view(b, n, H, nope + self.vdim)
        # token-major buffers: q (rotary slice rotated), k (per-head nope part | the shared
        # rotated key), v (zero columns past v_head_dim)
        qb = torch.cat((q[..., :nope], self.rotary.rotate(q[..., nope:], pos)), dim=-1)
        kb = torch.empty((b, n, H, w), dtype=x.dtype, device=x.device)
        kb[..., :nope] = kv[..., :nope]
        kb[..., nope:] = self.rotary.rotate(k_rot, pos).unsqueeze(2)
        vb = kv.new_zeros((b, n, H, w))
        vb[..., : self.vdim] = kv[..., nope:]
        qh, kh, vh = (t.transpose(1, 2) for t in (qb, kb, vb))  # [b, H, n, w] views
        if attention_mask is None:
            o = F.scaled_dot_product_attention(qh, kh, vh, is_causal=True, scale=self.scale)
        else:
            o = F.scaled_dot_product_attention(qh, kh, vh, attn_mask=attention_mask.to(x.dtype), scale=self.scale)
        return self.o_proj(o.transpose(1, 2)[..., : self.vdim].reshape(b, n, H * self.vdim))


class FFN(nn.Module):
    """SwiGLU feed-forward of the dense blocks, w2(silu(w1 x) * (w3 x)) (model.py:257-265),
    with the gate and up projections as one GEMM over their stacked weights."""

    def __init__(self, config):
        super().__init__()
        self.w1 = nn.Linear(config.d_model, config.d_ffn_intermediate, bias=False)
        self.w2 = nn.Linear(config.d_ffn_intermediate, config.d_model, bias=False)
        self.w3 = nn.Linear(config.d_model, config.d_ffn_intermediate, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate, up = F.linear(x, _stacked(self, (self.w1, self.w3))).chunk(2, dim=-1)
        return self.w2(F.silu(gate) * up)


class TransformerBlock(nn.Module):
    """Pre-norm residual block: h = x + attn(norm1(x)); out = h + mlp(norm2(h))
    (model.py:345-365)."""

    def __init__(self, config, is_moe_layer: bool):
        super().__init__()
        self.self_attn = MLAttention(config)
        self.mlp = EthosExpertLayer(config) if is_moe_layer else FFN(config)
        self.input_layernorm = RMSNorm(config.d_model, eps=config.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(config.d_model, eps=config.rms_norm_eps)

    def forward(self, x, attention_mask, position_ids):
        h = x + self.self_attn(self.input_layernorm(x), attention_mask, position_ids)
        return h + self.mlp(self.post_attention_layernorm(h))


class CompressedMoEModel(nn.Module):
    """Token ids [batch, seq] -> logits [batch, seq, vocab] (model.py:367-396)."""

    def __init__(self, config):
        super().__init__()
        self.config = config
        self.tok_embeddings = nn.Embedding(config.vocab_size, config.d_model)
        self.layers = nn.ModuleList([TransformerBlock(config, i >= config.num_dense_layers)
                                     for i in range(config.num_layers)])
        self.norm = RMSNorm(config.d_model, eps=config.rms_norm_eps)
        self.output = nn.Linear(config.d_model, config.vocab_size, bias=False)
        self.output.weight = self.tok_embeddings.weight  # one matrix for embedding and head

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        seq = input_ids.shape[1]
        pos = torch.arange(seq, device=input_ids.device)
        h = self.tok_embeddings(input_ids)
        for block in self.layers:
            h = block(h, None, pos)  # None: causal attention
        return self.output(self.norm(h))


def init_random_(model: CompressedMoEModel, seed: int = 0) -> CompressedMoEModel:
    """Random initialisation on the CPU with the expert layers' benchmark distributions
    (latents N(0, 0.02), sub-keys N(0, 1/sqrt(d_query/2)), nn.Linear defaults elsewhere)."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("expert_latents.weight"):
                p.copy_(torch.randn(p.shape, generator=g) * 0.02)
            elif ".sub_keys_" in name:
                p.copy_(torch.randn(p.shape, generator=g) / math.sqrt(p.shape[1]))
            elif name.endswith("layernorm.weight") or name.endswith("norm.weight") or "query_norms" in name:
                if "query_norms" in name and name.endswith("bias"):
                    p.zero_()
                else:
                    p.fill_(1.0)
            elif p.dim() == 2:
                bound = 1.0 / math.sqrt(p.shape[1])
                p.copy_((torch.rand(p.shape, generator=g) * 2 - 1) * bound)
            else:
                bound = 1.0 / math.sqrt(p.shape[0])
                p.copy_((torch.rand(p.shape, generator=g) * 2 - 1) * bound)
    return model
