"""The language model's module tree against the reference's (CompressedMoEModel,
model.py:345-396): state_dict keys, tied head, checkpoint helpers.  CPU only."""
import torch

from ethos_amd import checkpoint as ck
from ethos_amd.layer import EthosExpertLayer
from ethos_amd.model import CompressedMoEModel, FFN, init_random_, lm_config

TINY = dict(vocab_size=500, d_model=64, num_layers=3, num_heads=4, num_dense_layers=1, q_lora_rank=48,
            kv_lora_rank=32, v_head_dim=16, qk_nope_head_dim=16, qk_rope_head_dim=16, num_experts=256, d_latent=16,
            d_intermediate_hypernet=32, top_k=4, num_routing_heads=2, d_query=32, d_ffn_intermediate=128,
            max_seq_len=64)

# per-block keys of the reference (model.py:79-100 attention, 257-265 FFN, 345-360 block)
ATTN = ["q_a_proj.weight", "q_a_layernorm.weight", "q_b_proj.weight", "kv_a_proj_with_mqa.weight",
        "kv_a_layernorm.weight", "kv_b_proj.weight", "o_proj.weight"]


def test_state_dict_layout_matches_reference():
    cfg = lm_config(**TINY)
    m = CompressedMoEModel(cfg)
    keys = set(m.state_dict().keys())
    want = {"tok_embeddings.weight", "norm.weight", "output.weight"}
    for i in range(cfg.num_layers):
        p = f"layers.{i}."
        want |= {p + "self_attn." + k for k in ATTN}
        want |= {p + "input_layernorm.weight", p + "post_attention_layernorm.weight"}
        if i < cfg.num_dense_layers:
            want |= {p + "mlp.w1.weight", p + "mlp.w2.weight", p + "mlp.w3.weight"}
        else:
            want |= {p + "mlp." + k for k in EthosExpertLayer(cfg).state_dict()}
    assert keys == want
    assert m.output.weight is m.tok_embeddings.weight
    assert isinstance(m.layers[0].mlp, FFN) and isinstance(m.layers[1].mlp, EthosExpertLayer)
    shapes = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    assert shapes["layers.1.self_attn.q_b_proj.weight"] == (4 * 32, 48)
    assert shapes["layers.1.self_attn.kv_a_proj_with_mqa.weight"] == (32 + 16, 64)
    assert shapes["layers.1.self_attn.kv_b_proj.weight"] == (4 * (16 + 16), 32)
    assert shapes["layers.1.self_attn.o_proj.weight"] == (64, 4 * 16)


def test_checkpoint_round_trip_and_expert_prefixes():
    cfg = lm_config(**TINY)
    a = init_random_(CompressedMoEModel(cfg), seed=3)
    b = CompressedMoEModel(cfg)
    b.load_state_dict(a.state_dict(), strict=True)
    for k, v in a.state_dict().items():
        assert torch.equal(v, b.state_dict()[k]), k
    assert ck.expert_layer_prefixes(a.state_dict()) == ["layers.1.mlp.", "layers.2.mlp."]
    assert ck.replace_expert_layers(a) == []
