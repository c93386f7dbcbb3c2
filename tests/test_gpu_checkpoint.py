"""Checkpoint interop on the GPU.  The reference loads whole-model state_dicts
(notebooks/demo.ipynb:54-58) and saves DeepSpeed checkpoints (train.py:257-260); its Query
BatchNorm is an nn.BatchNorm1d (model.py:200-202) that updates its running statistics in
training mode.  Here:

  - reference-format checkpoints written to disk (a whole-model pytorch_model.bin, and a
    DeepSpeed checkpoint directory with "module."-prefixed keys under its tag directory) are
    read by ethos_amd.checkpoint, every expert layer they hold is built on the GPU and run
    through the HIP path against the oracle (fp32 and bf16), and the whole small model loaded
    from them reproduces the reference's own logits (tests/golden/lm_tiny.npz);
  - reference-structured modules are swapped in place by replace_expert_layers and run
    against the oracle;
  - a training-mode forward updates running_mean / running_var / num_batches_tracked as
    F.batch_norm does, normalises with the batch statistics, and the eval-mode layer then
    uses the updated statistics."""
import json
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch import nn

from ethos_amd import EthosExpertLayer, ExpertGenerationNetwork, ProductKeyRouter
from ethos_amd import checkpoint as ck
from ethos_amd.model import CompressedMoEModel
from ethos_amd.workloads import SHAPES, make_inputs, make_lm_inputs
from golden_util import GOLDEN
from gpu_util import check_out, to_host
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _write(tmp_path, sd):
    whole = tmp_path / "pytorch_model.bin"
    torch.save(sd, whole)
    tag = tmp_path / "ds_ckpt" / "global_step10"
    tag.mkdir(parents=True)
    # DeepSpeed's model-states file: the weights under "module", here with the "module."
    # key prefix a DDP-wrapped engine leaves, plus bookkeeping entries
    torch.save({"module": {"module." + k: v for k, v in sd.items()}, "global_steps": 10, "dp_world_size": 1},
               tag / "mp_rank_00_model_states.pt")
    (tmp_path / "ds_ckpt" / "latest").write_text("global_step10")
    return {"pytorch_model.bin": whole, "deepspeed": tmp_path / "ds_ckpt"}


def _check_layer(layer, n_heads, top_k, dt, seed):
    d = layer.d_model
    x = torch.randn((40, d), generator=torch.Generator().manual_seed(seed)).to(layer.expert_latents.weight.dtype)
    with torch.no_grad():
        y = layer(x.cuda().view(1, 40, d)).view(40, d)
    P = O.unpack_state({k: v.cpu() for k, v in layer.state_dict().items()}, n_heads)
    r = O.layer_forward(O.from_torch(x), P, n_heads, top_k, dt)
    gates, ids = layer.router(x.cuda())
    assert np.array_equal(ids.cpu().numpy(), r["ids"])
    check_out(O.to_f32(to_host(y), dt), r["out"], dt, signal=True, nerr_max=2e-3)


@pytest.mark.parametrize("fmt", ["pytorch_model.bin", "deepspeed"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_reference_checkpoints_run_through_hip_path(tmp_path, fmt, dtype):
    cfg, sd, _ = make_lm_inputs(seed=0)
    path = _write(tmp_path, sd)[fmt]
    loaded = ck.load_state_dict_file(path)
    assert set(loaded) == set(sd)
    prefixes = ck.expert_layer_prefixes(loaded)
    assert prefixes == ["layers.1.mlp.", "layers.2.mlp."]
    dt = "fp32" if dtype == torch.float32 else "bf16"
    for j, p in enumerate(prefixes):
        lsd = {k: (v.to(dtype) if v.is_floating_point() else v).cuda()
               for k, v in ck.expert_layer_state_dict(loaded, p).items()}
        layer = ck.layer_from_state_dict(lsd, top_k=cfg.top_k).eval()
        assert isinstance(layer, EthosExpertLayer) and layer.expert_latents.weight.is_cuda
        assert layer.expert_latents.weight.dtype == dtype
        _check_layer(layer, cfg.num_routing_heads, cfg.top_k, dt, seed=j)


@pytest.mark.parametrize("fmt", ["pytorch_model.bin", "deepspeed"])
def test_whole_model_from_checkpoint_reproduces_reference_logits(tmp_path, fmt):
    f = np.load(os.path.join(GOLDEN, "lm_tiny.npz"), allow_pickle=False)
    meta = json.loads(str(f["meta"]))
    cfg, sd, ids = make_lm_inputs(seed=meta["seed"], batch=meta["batch"], seq=meta["seq"])
    path = _write(tmp_path, sd)[fmt]
    m = CompressedMoEModel(cfg)
    m.load_state_dict(ck.load_state_dict_file(path), strict=True)
    m = m.cuda().eval()
    with torch.no_grad():
        logits = m(ids.cuda()).double().cpu()
    ref = torch.from_numpy(f["ref_logits_fp32"]).double()
    assert float((logits - ref).norm() / ref.norm()) < 1e-4


class _RefShapedLayer(nn.Module):
    """The attribute set and submodule layout of the reference's expert layers
    (SimplifiedHypernetMoE, model.py:266-287), which is all replace_expert_layers reads."""

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


def test_replace_expert_layers_in_place_then_run(tmp_path):
    cfg, sd, _ = make_lm_inputs(seed=0)
    host = nn.ModuleDict({"a": _RefShapedLayer(cfg), "b": nn.Linear(4, 4), "c": _RefShapedLayer(cfg)})
    layer_sds = [ck.expert_layer_state_dict(sd, p) for p in ("layers.1.mlp.", "layers.2.mlp.")]
    torch.save({"a." + k: v for k, v in layer_sds[0].items()} | {"c." + k: v for k, v in layer_sds[1].items()}
               | {"b.weight": torch.eye(4), "b.bias": torch.zeros(4)}, tmp_path / "host.bin")
    assert ck.replace_expert_layers(host) == ["a", "c"]
    host.load_state_dict(ck.load_state_dict_file(tmp_path / "host.bin"), strict=True)
    host = host.cuda().eval()
    for j, name in enumerate(("a", "c")):
        assert isinstance(host[name], EthosExpertLayer)
        _check_layer(host[name], cfg.num_routing_heads, cfg.top_k, "fp32", seed=10 + j)


def test_train_mode_batchnorm_updates_running_stats():
    sh = SHAPES["cfg1"]  # fp32, 256 tokens, 4 heads
    x, sd = make_inputs(sh, signal=True)
    g = torch.Generator().manual_seed(5)
    for h in range(sh.num_heads):  # non-trivial starting statistics and affine parameters
        sd[f"router.query_norms.{h}.running_mean"] = torch.randn(sh.d_query, generator=g) * 0.1
        sd[f"router.query_norms.{h}.running_var"] = torch.rand(sh.d_query, generator=g) + 0.5
        sd[f"router.query_norms.{h}.weight"] = torch.rand(sh.d_query, generator=g) + 0.5
        sd[f"router.query_norms.{h}.bias"] = torch.randn(sh.d_query, generator=g) * 0.1
    layer = EthosExpertLayer(sh.config())
    layer.load_state_dict(sd)
    layer = layer.cuda().train()
    xd = x.cuda()
    steps = 2
    with torch.no_grad():
        for _ in range(steps):
            q_train = layer.router.queries(xd)
            y = layer(xd.view(sh.batch, -1, sh.d_model))
    assert bool(torch.isfinite(y).all())
    # expected: F.batch_norm's update, applied `steps` times per head, in float64 on the CPU
    xx = x.double()
    for h in range(sh.num_heads):
        pre = f"router.query_norms.{h}."
        q = xx @ sd[f"router.query_projs.{h}.weight"].double().T + sd[f"router.query_projs.{h}.bias"].double()
        rm, rv = sd[pre + "running_mean"].double().clone(), sd[pre + "running_var"].double().clone()
        for _ in range(2 * steps):  # queries() and the forward each update the statistics once
            F.batch_norm(q, rm, rv, None, None, True, 0.1, 1e-5)
        m = layer.router.query_norms[h]
        np.testing.assert_allclose(m.running_mean.double().cpu().numpy(), rm.numpy(), rtol=1e-5, atol=1e-7)
        np.testing.assert_allclose(m.running_var.double().cpu().numpy(), rv.numpy(), rtol=1e-5, atol=1e-7)
        assert int(m.num_batches_tracked) == 2 * steps
        # normalised with the batch statistics (biased variance) and the affine parameters
        qn = F.batch_norm(q, None, None, sd[pre + "weight"].double(), sd[pre + "bias"].double(), True, 0.1, 1e-5)
        np.testing.assert_allclose(q_train[:, h].double().cpu().numpy(), qn.numpy(), rtol=1e-4, atol=1e-5)
    # eval mode afterwards: the projection uses the updated running statistics, exactly as
    # the oracle's eval BatchNorm with those statistics
    layer.eval()
    with torch.no_grad():
        q_eval = layer.router.queries(xd)
    P = O.unpack_state({k: v.cpu() for k, v in layer.state_dict().items()}, sh.num_heads)
    want = O.query_proj(O.from_torch(x), P["Wq"], P["bq"], P["alpha"], P["beta"], "fp32")
    assert np.array_equal(to_host(q_eval), want)
