"""Checkpoint interop (host logic, CPU): reference-shaped state_dicts and modules into the
drop-in layer.  The reference classes themselves are not imported; `RefExpertLayer` below has
their attribute set and submodule structure (model.py:266-287), which is all the interop reads."""
import os
from types import SimpleNamespace

import pytest
import torch
from torch import nn

from ethos_amd import EthosExpertLayer, ExpertGenerationNetwork, ProductKeyRouter
from ethos_amd import checkpoint as ck

CFG = SimpleNamespace(d_model=32, num_experts=16, top_k=2, num_routing_heads=2, d_latent=8,
                      d_intermediate_hypernet=16, d_query=8)


class RefExpertLayer(nn.Module):
    """Attribute set and parameter layout of the reference's SimplifiedHypernetMoE."""

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


class FFN(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.w1 = nn.Linear(d, 2 * d, bias=False)


class Block(nn.Module):
    def __init__(self, mlp):
        super().__init__()
        self.norm = nn.LayerNorm(CFG.d_model)
        self.mlp = mlp


class ToyModel(nn.Module):
    """layers.0 dense, layers.1 and layers.2 expert layers (model.py:368-378 layout)."""

    def __init__(self):
        super().__init__()
        self.embed = nn.Embedding(10, CFG.d_model)
        self.layers = nn.ModuleList([Block(FFN(CFG.d_model)), Block(RefExpertLayer(CFG)), Block(RefExpertLayer(CFG))])


def _randomize(model):
    g = torch.Generator().manual_seed(0)
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(torch.randn(p.shape, generator=g))
        for name, b in model.named_buffers():
            if b.is_floating_point():
                b.copy_(torch.rand(b.shape, generator=g) + 0.5)
            else:
                b.fill_(7)
    return model


def test_normalize_state_dict_wrappers():
    sd = {"a.weight": torch.ones(2), "b.bias": torch.zeros(3)}
    assert ck.normalize_state_dict(sd).keys() == sd.keys()
    ds = {"module": sd, "buffer_names": ["x"], "global_steps": 10}
    assert ck.normalize_state_dict(ds).keys() == sd.keys()
    pref = {"module." + k: v for k, v in sd.items()}
    assert ck.normalize_state_dict(pref).keys() == sd.keys()
    assert ck.normalize_state_dict({"state_dict": pref}).keys() == sd.keys()
    with pytest.raises(TypeError):
        ck.normalize_state_dict([1, 2])


@pytest.mark.parametrize("layout", ["pytorch_model.bin", "deepspeed_dir"])
def test_whole_model_checkpoint_slices_into_layers(tmp_path, layout):
    model = _randomize(ToyModel())
    full = model.state_dict()
    if layout == "pytorch_model.bin":
        path = tmp_path / "pytorch_model.bin"
        torch.save(full, path)
    else:
        path = tmp_path / "epoch_1"
        os.makedirs(path / "global_step10")
        torch.save({"module": full, "buffer_names": [], "global_steps": 10},
                   path / "global_step10" / "mp_rank_00_model_states.pt")
    sd = ck.load_state_dict_file(path)
    assert ck.expert_layer_prefixes(sd) == ["layers.1.mlp.", "layers.2.mlp."]
    for i in (1, 2):
        layer_sd = ck.expert_layer_state_dict(sd, f"layers.{i}.mlp.")
        cfg = ck.config_from_state_dict(layer_sd, top_k=CFG.top_k)
        assert vars(cfg) == vars(CFG)
        layer = ck.layer_from_state_dict(layer_sd, top_k=CFG.top_k)
        assert isinstance(layer, EthosExpertLayer)
        ref_sd = model.layers[i].mlp.state_dict()
        got = layer.state_dict()
        assert got.keys() == ref_sd.keys()
        for k in ref_sd:
            assert torch.equal(got[k], ref_sd[k]), k


def test_config_needs_query_projections():
    with pytest.raises(KeyError):
        ck.config_from_state_dict({"expert_latents.weight": torch.zeros(4, 2)}, top_k=1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_replace_expert_layers_in_place(dtype):
    model = _randomize(ToyModel()).to(dtype)
    model.layers[2].mlp.train(False)
    before = {k: v.clone() for k, v in model.state_dict().items()}
    names = ck.replace_expert_layers(model)
    assert names == ["layers.1.mlp", "layers.2.mlp"]
    assert isinstance(model.layers[1].mlp, EthosExpertLayer) and isinstance(model.layers[2].mlp, EthosExpertLayer)
    assert isinstance(model.layers[0].mlp, FFN)
    assert model.layers[1].mlp.training and not model.layers[2].mlp.training
    assert model.layers[1].mlp.top_k == CFG.top_k
    after = model.state_dict()
    assert after.keys() == before.keys()
    for k in before:
        assert after[k].dtype == before[k].dtype and torch.equal(after[k], before[k]), k
    # a reference checkpoint still loads strictly into the converted model
    model.load_state_dict(before, strict=True)
    assert ck.replace_expert_layers(model) == []
