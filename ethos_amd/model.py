"""The ETHOS language model around the drop-in expert layer (the whole-model forward).

Module tree, constructor attributes and state_dict keys follow the reference's
CompressedMoEModel (model.py:367-396): token embedding tied to the output head, blocks of
pre-norm MLA attention (model.py:79-165) and an expert layer (or, for the first
num_dense_layers blocks, the SwiGLU FFN of model.py:257-265), a final RMSNorm.  A
reference checkpoint therefore loads with load_state_dict(strict=True).

The expert layer is EthosExpertLayer (HIP kernels); attention runs on
torch.nn.functional.scaled_dot_product_attention with a causal mask, which computes the
reference's masked softmax(QK^T * scale) V (model.py:156-163; its flash-attention branch,
model.py:133-155, pads V to the QK head width the same way this module does).  Inputs live
on a HIP device.
"""
from __future__ import annotations

import math
from types import SimpleNamespace

import torch
import torch.nn as nn
import torch.nn.functional as F

from .layer import EthosExpertLayer

# configs/default.yaml of the reference, with the expert-layer shape of the benchmarked
# layer (d_query 256) and the 12-block, all-expert-layer depth of the whole-model workload
LM_DEFAULTS = dict(vocab_size=100277, d_model=1024, num_layers=12, num_heads=16, num_dense_layers=0,
                   q_lora_rank=768, kv_lora_rank=256, v_head_dim=64, qk_nope_head_dim=64, qk_rope_head_dim=64,
                   num_experts=262144, d_latent=128, d_intermediate_hypernet=512, top_k=16, num_routing_heads=8,
                   d_query=256, d_ffn_intermediate=4096, max_seq_len=4096, rms_norm_eps=1e-6, rope_theta=10000.0)


def lm_config(**overrides) -> SimpleNamespace:
    cfg = dict(LM_DEFAULTS)
    cfg.update(overrides)
    return SimpleNamespace(**cfg)


class RMSNorm(nn.Module):
    """weight * RN_T(x / sqrt(mean(x^2) + eps)) with the statistics in float32
    (DeepseekV3RMSNorm, model.py:19-30)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        dt = x.dtype
        xf = x.to(torch.float32)
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.variance_epsilon)
        return self.weight * xf.to(dt)


class RotaryEmbedding(nn.Module):
    """cos / sin tables of the rotary position embedding (model.py:33-59): frequencies
    base^(-2i/dim), each repeated for both halves of the rotated dimension."""

    def __init__(self, dim: int, max_position_embeddings: int = 2048, base: float = 10000.0):
        super().__init__()
        self.dim = dim
        self.base = base
        inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2).float() / dim))
        self.register_buffer("inv_freq", inv_freq, persistent=False)
        self._cache = None
        self._cache_len = max_position_embeddings

    def forward(self, x: torch.Tensor, seq_len: int):
        n = max(seq_len, self._cache_len)
        c = self._cache
        if c is None or c[0].shape[0] < seq_len or c[0].device != x.device:
            t = torch.arange(n, device=x.device, dtype=torch.float32)
            freqs = torch.outer(t, self.inv_freq.to(x.device))
            emb = torch.cat((freqs, freqs), dim=-1)
            # the reference builds its tables in the default dtype (float32) and casts per call
            c = self._cache = (emb.cos(), emb.sin())
        return c[0][:seq_len].to(x.dtype), c[1][:seq_len].to(x.dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rotary(q, k, cos, sin, position_ids):
    """(q cos + rot(q) sin, k cos + rot(k) sin) at the given positions (model.py:68-76)."""
    if position_ids.dim() == 1:
        position_ids = position_ids.unsqueeze(0)
    cos = cos[position_ids].unsqueeze(1)
    sin = sin[position_ids].unsqueeze(1)
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


class MLAttention(nn.Module):
    """Multi-head latent attention (DeepseekV3Attention, model.py:79-165): queries through a
    low-rank projection with RMSNorm, keys and values from a compressed KV latent plus one
    shared rotary key, causal softmax attention with scale q_head_dim^-1/2."""

    def __init__(self, config):
        super().__init__()
        self.hidden_size = config.d_model
        self.num_heads = config.num_heads
        self.q_lora_rank = config.q_lora_rank
        self.qk_rope_head_dim = config.qk_rope_head_dim
        self.kv_lora_rank = config.kv_lora_rank
        self.v_head_dim = config.v_head_dim
        self.qk_nope_head_dim = config.qk_nope_head_dim
        self.q_head_dim = config.qk_nope_head_dim + config.qk_rope_head_dim
        self.q_a_proj = nn.Linear(self.hidden_size, config.q_lora_rank, bias=False)
        self.q_a_layernorm = RMSNorm(config.q_lora_rank, eps=config.rms_norm_eps)
        self.q_b_proj = nn.Linear(config.q_lora_rank, self.num_heads * self.q_head_dim, bias=False)
        self.kv_a_proj_with_mqa = nn.Linear(self.hidden_size, config.kv_lora_rank + config.qk_rope_head_dim,
                                            bias=False)
        self.kv_a_layernorm = RMSNorm(config.kv_lora_rank, eps=config.rms_norm_eps)
        self.kv_b_proj = nn.Linear(config.kv_lora_rank,
                                   self.num_heads * (self.qk_nope_head_dim + self.v_head_dim), bias=False)
        self.o_proj = nn.Linear(self.num_heads * self.v_head_dim, self.hidden_size, bias=False)
        self.rotary_emb = RotaryEmbedding(self.qk_rope_head_dim, config.max_seq_len, config.rope_theta)
        self.softmax_scale = self.q_head_dim ** (-0.5)

    def forward(self, hidden_states: torch.Tensor, attention_mask, position_ids: torch.Tensor) -> torch.Tensor:
        """`attention_mask`: None for causal attention, else an additive [seq, seq] mask (the
        reference passes triu(-inf, 1), model.py:389-390, which is the causal case)."""
        b, n, _ = hidden_states.shape
        H = self.num_heads
        q = self.q_b_proj(self.q_a_layernorm(self.q_a_proj(hidden_states))).view(b, n, H, self.q_head_dim)
        q_nope, q_pe = torch.split(q, [self.qk_nope_head_dim, self.qk_rope_head_dim], dim=-1)
        ckv = self.kv_a_proj_with_mqa(hidden_states)
        ckv, k_pe = torch.split(ckv, [self.kv_lora_rank, self.qk_rope_head_dim], dim=-1)
        k_pe = k_pe.view(b, n, 1, self.qk_rope_head_dim)
        kv = self.kv_b_proj(self.kv_a_layernorm(ckv)).view(b, n, H, self.qk_nope_head_dim + self.v_head_dim)
        k_nope, v = torch.split(kv, [self.qk_nope_head_dim, self.v_head_dim], dim=-1)
        cos, sin = self.rotary_emb(v, n)
        q_pe, k_pe = apply_rotary(q_pe.transpose(1, 2), k_pe.transpose(1, 2), cos, sin, position_ids)
        q = torch.cat([q_nope.transpose(1, 2), q_pe], dim=-1).contiguous()
        k = torch.cat([k_nope.transpose(1, 2), k_pe.expand(b, H, n, self.qk_rope_head_dim)], dim=-1).contiguous()
        v = v.transpose(1, 2)
        if self.v_head_dim != self.q_head_dim:
            v = F.pad(v, [0, self.q_head_dim - self.v_head_dim])
        if attention_mask is None:
            o = F.scaled_dot_product_attention(q, k, v.contiguous(), is_causal=True, scale=self.softmax_scale)
        else:
            o = F.scaled_dot_product_attention(q, k, v.contiguous(), attn_mask=attention_mask.to(q.dtype),
                                               scale=self.softmax_scale)
        o = o[..., : self.v_head_dim].transpose(1, 2).reshape(b, n, H * self.v_head_dim)
        return self.o_proj(o)


class FFN(nn.Module):
    """SwiGLU feed-forward of the dense blocks: w2(silu(w1 x) * w3 x) (model.py:257-265)."""

    def __init__(self, config):
        super().__init__()
        self.w1 = nn.Linear(config.d_model, config.d_ffn_intermediate, bias=False)
        self.w2 = nn.Linear(config.d_ffn_intermediate, config.d_model, bias=False)
        self.w3 = nn.Linear(config.d_model, config.d_ffn_intermediate, bias=False)

    def forward(self, x):
        return self.w2(F.silu(self.w1(x)) * self.w3(x))


class TransformerBlock(nn.Module):
    """h = x + attn(norm(x)); out = h + mlp(norm(h)) (model.py:345-365)."""

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
        self.tok_embeddings.weight = self.output.weight

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        _, seq_len = input_ids.shape
        h = self.tok_embeddings(input_ids)
        position_ids = torch.arange(seq_len, dtype=torch.long, device=input_ids.device)
        for layer in self.layers:
            h = layer(h, None, position_ids)  # None: causal, as the reference's triu(-inf, 1) mask
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
