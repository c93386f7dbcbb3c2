"""Checkpoint interop: reference state_dicts into the drop-in expert layer.

The reference trains with DeepSpeed (`model_engine.save_checkpoint`, train.py:257-260) and
loads a consolidated `pytorch_model.bin` into `CompressedMoEModel` with
`model.load_state_dict` (notebooks/demo.ipynb, "Load checkpoint" cell).  Expert layers sit at
`layers.{i}.mlp` for i >= num_dense_layers (model.py:345-378), and both reference classes
(SimplifiedHypernetMoE, model.py:266-287; FusedLowRankMoE_Reordered, kernels.py:125-145)
carry the state_dict keys that `EthosExpertLayer` shares, so a whole-model checkpoint loads
unchanged into a model whose expert layers were replaced, and one layer's slice loads into
a standalone `EthosExpertLayer`.

Files are read with `torch.load(..., weights_only=True)`: nothing in a checkpoint is executed.
"""
from __future__ import annotations

import os
import re
from types import SimpleNamespace

import torch
from torch import nn

from .layer import EthosExpertLayer

# Keys every expert layer has (besides the per-head query projections and norms).
LAYER_KEYS = (
    "expert_latents.weight",
    "generation_network.net.0.weight",
    "generation_network.net.2.weight",
    "router.sub_keys_1.weight",
    "router.sub_keys_2.weight",
)

_LAYER_INDEX = re.compile(r"(\d+)")


def normalize_state_dict(obj) -> dict:
    """A flat name -> tensor dict from what a checkpoint file holds.

    Accepts a plain state_dict (`pytorch_model.bin`), a DeepSpeed model-states dict (the
    weights under "module", other entries ignored) or a {"state_dict": ...} wrapper, and
    removes a "module." prefix that DDP / DeepSpeed wrappers put on every key."""
    if isinstance(obj, dict):
        for key in ("module", "state_dict", "model"):
            inner = obj.get(key)
            if isinstance(inner, dict) and any(torch.is_tensor(v) for v in inner.values()):
                obj = inner
                break
    if not isinstance(obj, dict):
        raise TypeError(f"checkpoint holds {type(obj).__name__}, not a state_dict")
    sd = {k: v for k, v in obj.items() if torch.is_tensor(v)}
    if sd and all(k.startswith("module.") for k in sd):
        sd = {k[len("module."):]: v for k, v in sd.items()}
    return sd


def load_state_dict_file(path: str | os.PathLike, map_location="cpu") -> dict:
    """`torch.load(path, weights_only=True)`, normalised as by `normalize_state_dict`.

    A DeepSpeed checkpoint directory (`save_checkpoint` output) is accepted too: its
    `mp_rank_00_model_states.pt` (possibly one level down, under the tag directory) is read."""
    path = os.fspath(path)
    if os.path.isdir(path):
        found = None
        for root, _dirs, files in os.walk(path):
            if "mp_rank_00_model_states.pt" in files:
                found = os.path.join(root, "mp_rank_00_model_states.pt")
                break
        if found is None:
            raise FileNotFoundError(f"no mp_rank_00_model_states.pt under {path}")
        path = found
    return normalize_state_dict(torch.load(path, map_location=map_location, weights_only=True))


def expert_layer_prefixes(state_dict: dict) -> list[str]:
    """Prefixes P (e.g. "layers.2.mlp.") such that P + every expert-layer key is present,
    ordered by the first layer index in P (then lexically)."""
    cands = {k[: -len(LAYER_KEYS[0])] for k in state_dict if k.endswith(LAYER_KEYS[0])}
    found = [p for p in cands if all(p + k in state_dict for k in LAYER_KEYS)]

    def order(p: str):
        m = _LAYER_INDEX.search(p)
        return (int(m.group(1)) if m else -1, p)

    return sorted(found, key=order)


def expert_layer_state_dict(state_dict: dict, prefix: str) -> dict:
    """The keys under `prefix`, with the prefix removed."""
    return {k[len(prefix):]: v for k, v in state_dict.items() if k.startswith(prefix)}


def config_from_state_dict(layer_sd: dict, top_k: int) -> SimpleNamespace:
    """The constructor config of one expert layer, read from its parameter shapes.

    `top_k` is not stored in a state_dict (the reference takes it from its config) and must
    be given."""
    n_heads = 0
    while f"router.query_projs.{n_heads}.weight" in layer_sd:
        n_heads += 1
    if n_heads == 0:
        raise KeyError("no router.query_projs.{h}.weight in the layer state_dict")
    d_query, d_model = layer_sd["router.query_projs.0.weight"].shape
    num_experts, d_latent = layer_sd["expert_latents.weight"].shape
    d_hidden = layer_sd["generation_network.net.0.weight"].shape[0]
    if layer_sd["generation_network.net.2.weight"].shape != (2 * d_model, d_hidden):
        raise ValueError("generation_network.net.2.weight is not [2 d_model, d_hidden]")
    return SimpleNamespace(d_model=int(d_model), num_experts=int(num_experts), top_k=int(top_k),
                           num_routing_heads=n_heads, d_latent=int(d_latent),
                           d_intermediate_hypernet=int(d_hidden), d_query=int(d_query))


def layer_from_state_dict(layer_sd: dict, top_k: int) -> EthosExpertLayer:
    """A new `EthosExpertLayer` holding `layer_sd` (strict load), on the tensors' device and
    in their floating dtype."""
    layer = EthosExpertLayer(config_from_state_dict(layer_sd, top_k))
    ref = layer_sd["expert_latents.weight"]
    layer = layer.to(device=ref.device, dtype=ref.dtype)
    layer.load_state_dict(layer_sd, strict=True)
    return layer


def _is_reference_expert_layer(mod: nn.Module) -> bool:
    return (not isinstance(mod, EthosExpertLayer) and all(hasattr(mod, a) for a in (
        "router", "expert_latents", "generation_network", "d_model", "num_experts", "top_k", "num_heads",
        "d_latent", "d_hidden")))


def replace_expert_layers(model: nn.Module) -> list[str]:
    """Swap every reference expert layer inside `model` (a module with the attribute set of
    SimplifiedHypernetMoE / FusedLowRankMoE_Reordered) for an `EthosExpertLayer` carrying
    the same parameters and buffers, device, dtype and train/eval mode.  Returns the
    qualified names replaced.  Afterwards `model.load_state_dict` of a reference checkpoint
    works unchanged."""
    replaced = []
    for name, mod in list(model.named_modules()):
        if not name or not _is_reference_expert_layer(mod):
            continue
        cfg = SimpleNamespace(d_model=mod.d_model, num_experts=mod.num_experts, top_k=mod.top_k,
                              num_routing_heads=mod.num_heads, d_latent=mod.d_latent,
                              d_intermediate_hypernet=mod.d_hidden,
                              d_query=mod.router.query_projs[0].out_features)
        ref = mod.expert_latents.weight
        new = EthosExpertLayer(cfg).to(device=ref.device, dtype=ref.dtype)
        new.load_state_dict(mod.state_dict(), strict=True)
        new.train(mod.training)
        parent_name, _, attr = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        setattr(parent, attr, new)
        replaced.append(name)
    return replaced
