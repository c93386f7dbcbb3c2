"""Seeded synthetic workloads for the ETHOS expert layer.

Shapes are the expert-layer configurations the benchmarks and parity tests use;
parameters are drawn in a fixed order from one ``torch.Generator('cpu')`` so every
machine regenerates identical inputs:

    x, expert latents, generator W1, generator W2, {Wq_h, b_h} for h < H, sub-keys 1, 2

Distributions: x ~ N(0, 1); latents ~ N(0, 0.02); sub-keys ~ N(0, 1/sqrt(d_query/2));
Wq, b, W1, W2 ~ U(-1/sqrt(fan_in), 1/sqrt(fan_in)) (the nn.Linear default bound);
Query BatchNorm at running mean 0, running var 1, weight 1, bias 0.  Values are
drawn in fp32 and then cast to the layer dtype.

The returned dict uses the reference layer's state_dict names
(model.py:282-286 expert_latents / generation_network / router; model.py:195-206
query_projs / query_norms / sub_keys_{1,2}), so the same dict loads into the
reference module and into :class:`ethos_amd.EthosExpertLayer`.
"""
from __future__ import annotations

import dataclasses
import math
from types import SimpleNamespace

import torch


@dataclasses.dataclass(frozen=True)
class LayerShape:
    name: str
    n_tok: int
    d_model: int
    num_experts: int
    num_heads: int
    top_k: int
    d_query: int
    d_latent: int = 128
    d_hidden: int = 512
    dtype: str = "bf16"  # "fp32" | "bf16"
    batch: int = 1  # x is [batch, n_tok // batch, d_model]
    skew: float | None = None  # Zipf exponent applied to sub-key rows

    @property
    def n_sub(self) -> int:
        return math.isqrt(self.num_experts)

    @property
    def n_pairs(self) -> int:
        return self.n_tok * self.num_heads * self.top_k

    @property
    def torch_dtype(self) -> torch.dtype:
        return {"fp32": torch.float32, "bf16": torch.bfloat16}[self.dtype]

    def config(self) -> SimpleNamespace:
        """The attribute bag the layer constructor reads (model.py:275-280,185-189)."""
        return SimpleNamespace(
            d_model=self.d_model,
            num_experts=self.num_experts,
            top_k=self.top_k,
            num_routing_heads=self.num_heads,
            d_latent=self.d_latent,
            d_intermediate_hypernet=self.d_hidden,
            d_query=self.d_query,
        )

    def with_tokens(self, n_tok: int, batch: int = 1) -> "LayerShape":
        return dataclasses.replace(self, n_tok=n_tok, batch=batch)


SHAPES = {
    # 256 tokens (2 x 128), d 256, 4,096 experts, 4 heads, top-8, fp32.  The
    # configuration names both a 256->256 query projection and 64-wide sub-keys,
    # which the reference cannot have at once (sub-key width = d_query / 2), so
    # both readings are kept.
    "cfg1": LayerShape("cfg1", 256, 256, 4096, 4, 8, 256, dtype="fp32", batch=2),
    "cfg1_dq128": LayerShape("cfg1_dq128", 256, 256, 4096, 4, 8, 128, dtype="fp32", batch=2),
    # 4,096 tokens (2 x 2048), d 1024, 262,144 experts, 8 heads, top-16, bf16.
    "cfg2": LayerShape("cfg2", 4096, 1024, 262144, 8, 16, 256, batch=2),
    # 64 tokens, same layer (decode-like, low reuse).
    "cfg3": LayerShape("cfg3", 64, 1024, 262144, 8, 16, 256),
    # 32,768 tokens (16 x 2048), Zipf(1.1)-skewed sub-key rows.
    "cfg4": LayerShape("cfg4", 32768, 1024, 262144, 8, 16, 256, batch=16, skew=1.1),
    # The reference's default YAML layer shape (d_query 512 -> 256-wide sub-keys).
    "yaml": LayerShape("yaml", 256, 1024, 262144, 8, 16, 512),
    # Small shapes for fast tests.
    "tiny": LayerShape("tiny", 48, 64, 256, 2, 4, 32, d_latent=16, d_hidden=32, batch=2),
    "tiny_fp32": LayerShape("tiny_fp32", 48, 64, 256, 2, 4, 32, d_latent=16, d_hidden=32, dtype="fp32", batch=2),
}


def _uniform(gen: torch.Generator, shape, fan_in: int) -> torch.Tensor:
    bound = 1.0 / math.sqrt(fan_in)
    return (torch.rand(shape, generator=gen) * 2.0 - 1.0) * bound


def make_inputs(shape: LayerShape, seed: int = 0, signal: bool = False):
    """Return ``(x, state_dict)`` as CPU tensors in the layer dtype.

    ``signal=True`` draws latents from N(0, 1) and scales W1, W2 by 4 so the layer
    output is O(1e-2..1e-1) instead of O(1e-5); used for numerics checks only.
    """
    g = torch.Generator(device="cpu").manual_seed(seed)
    d, H, dq = shape.d_model, shape.num_heads, shape.d_query
    E, dl, dh = shape.num_experts, shape.d_latent, shape.d_hidden
    K, dh2 = shape.n_sub, dq // 2

    x = torch.randn((shape.n_tok, d), generator=g)
    latents = torch.randn((E, dl), generator=g) * (1.0 if signal else 0.02)
    w1 = _uniform(g, (dh, dl), dl)
    w2 = _uniform(g, (2 * d, dh), dh)
    if signal:
        w1 = w1 * 4.0
        w2 = w2 * 4.0
    sd = {
        "expert_latents.weight": latents,
        "generation_network.net.0.weight": w1,
        "generation_network.net.2.weight": w2,
    }
    for h in range(H):
        sd[f"router.query_projs.{h}.weight"] = _uniform(g, (dq, d), d)
        sd[f"router.query_projs.{h}.bias"] = _uniform(g, (dq,), d)
    k1 = torch.randn((K, dh2), generator=g) * (1.0 / math.sqrt(dh2))
    k2 = torch.randn((K, dh2), generator=g) * (1.0 / math.sqrt(dh2))
    if shape.skew is not None:
        zipf = (torch.arange(K, dtype=torch.float32) + 1.0) ** (-shape.skew)
        k1 = k1 * zipf[:, None]
        k2 = k2 * zipf[:, None]
    sd["router.sub_keys_1.weight"] = k1
    sd["router.sub_keys_2.weight"] = k2
    for h in range(H):
        sd[f"router.query_norms.{h}.weight"] = torch.ones(dq)
        sd[f"router.query_norms.{h}.bias"] = torch.zeros(dq)
        sd[f"router.query_norms.{h}.running_mean"] = torch.zeros(dq)
        sd[f"router.query_norms.{h}.running_var"] = torch.ones(dq)
        sd[f"router.query_norms.{h}.num_batches_tracked"] = torch.zeros((), dtype=torch.long)
    dt = shape.torch_dtype
    x = x.to(dt)
    sd = {k: (v.to(dt) if v.is_floating_point() else v) for k, v in sd.items()}
    return x, sd


# A small whole language model (3 blocks: one dense SwiGLU block, two expert blocks) for
# parity checks of the model around the expert layer.  v_head_dim 16 differs from the
# 32-wide query/key heads, as in the reference's default configuration (64 vs 128).
LM_TINY = dict(vocab_size=500, d_model=64, num_layers=3, num_heads=4, num_dense_layers=1, q_lora_rank=48,
               kv_lora_rank=32, v_head_dim=16, qk_nope_head_dim=16, qk_rope_head_dim=16, num_experts=256,
               d_latent=16, d_intermediate_hypernet=32, top_k=4, num_routing_heads=2, d_query=32,
               d_ffn_intermediate=128, max_seq_len=64)


def make_lm_inputs(seed: int = 0, batch: int = 2, seq: int = 24, expert_scale: float = 50.0):
    """``(config, state_dict, token ids)`` of the small language model, on the CPU in
    float32.  Parameters come from ``ethos_amd.model.init_random_(seed)``; the expert
    latents are then scaled by ``expert_scale`` so that the expert layers' outputs are of
    the order of the residual stream (at the benchmark scale they are ~1e-5 and would not
    show in the logits).  Token ids are uniform over the vocabulary."""
    from .layer import EthosExpertLayer
    from .model import CompressedMoEModel, init_random_, lm_config

    cfg = lm_config(**LM_TINY)
    m = init_random_(CompressedMoEModel(cfg), seed=seed)
    with torch.no_grad():
        for block in m.layers:
            if isinstance(block.mlp, EthosExpertLayer):
                block.mlp.expert_latents.weight.mul_(expert_scale)
    ids = torch.randint(0, cfg.vocab_size, (batch, seq), generator=torch.Generator().manual_seed(seed))
    return cfg, {k: v.detach().clone() for k, v in m.state_dict().items()}, ids
