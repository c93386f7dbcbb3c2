"""The language model's module tree against the reference's (CompressedMoEModel,
model.py:345-396): state_dict keys, tied head, checkpoint helpers.  CPU only."""
import torch

from ethos_amd import checkpoint as ck
from ethos_amd.layer import EthosExpertLayer
from ethos_amd.model import CompressedMoEModel, FFN, init_random_, lm_config
from ethos_amd.workloads import LM_TINY, make_lm_inputs
from torch_reference import _attention, _rms

TINY = LM_TINY

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


def _nerr(a, b):
    return float((a.double() - b.double()).norm() / b.double().norm())


def test_dense_block_matches_restatement():
    """The first block (attention + dense FFN, no expert layer, so it runs on the CPU)
    against the float32 restatement of the reference's block (itself pinned to the
    reference's logits), at positions 0..n-1 and at shifted positions."""
    cfg, sd, ids = make_lm_inputs(seed=0)
    m = CompressedMoEModel(cfg)
    m.load_state_dict(sd)
    m.eval()
    blk = m.layers[0]
    P = {k: v.float() for k, v in sd.items()}
    x = P["tok_embeddings.weight"][ids]
    eps = cfg.rms_norm_eps
    with torch.no_grad():
        hh = x + _attention(P, "layers.0.self_attn.", _rms(x, P["layers.0.input_layernorm.weight"], eps), cfg)
        z = _rms(hh, P["layers.0.post_attention_layernorm.weight"], eps)
        mlp = torch.nn.functional.linear(
            torch.nn.functional.silu(torch.nn.functional.linear(z, P["layers.0.mlp.w1.weight"]))
            * torch.nn.functional.linear(z, P["layers.0.mlp.w3.weight"]), P["layers.0.mlp.w2.weight"])
        want = hh + mlp
        got = blk(x, None, torch.arange(ids.shape[1]))
        assert _nerr(got, want) < 1e-6
        # an explicit additive causal mask gives the same result as the causal flag
        mask = torch.triu(torch.full((ids.shape[1],) * 2, float("-inf")), diagonal=1)
        assert _nerr(blk(x, mask, torch.arange(ids.shape[1])), want) < 1e-6


def test_rotary_matches_duplicated_table_form():
    """The half-rotation equals x cos(t) + rot(x) sin(t) with the angle table duplicated over
    both halves and rot(x) = [-x2, x1], in float32 and bit-for-bit in bfloat16."""
    from ethos_amd.model import Rotary

    r = Rotary(16, 10000.0)
    g = torch.Generator().manual_seed(0)
    for dt in (torch.float32, torch.bfloat16):
        x = torch.randn((2, 40, 3, 16), generator=g).to(dt)
        pos = torch.arange(5, 45)
        inv = 1.0 / (10000.0 ** (torch.arange(0, 16, 2).float() / 16))
        ang = torch.outer(pos.float(), inv)
        emb = torch.cat((ang, ang), -1)
        cos, sin = emb.cos().to(dt)[None, :, None, :], emb.sin().to(dt)[None, :, None, :]
        rot = torch.cat((-x[..., 8:], x[..., :8]), -1)
        assert torch.equal(r.rotate(x, pos), x * cos + rot * sin)
