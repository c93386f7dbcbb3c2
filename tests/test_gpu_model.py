"""The language model (ethos_amd.model.CompressedMoEModel) on the GPU against a float32
restatement of the reference's model forward (tests/torch_reference.lm_forward: matmul +
additive-mask attention, model.py:103-165, 345-396) with each expert layer's routing
imposed from the GPU run."""
import pytest
import torch

from ethos_amd.layer import EthosExpertLayer
from ethos_amd.model import CompressedMoEModel, init_random_, lm_config
from test_model_cpu import TINY
from torch_reference import lm_forward

pytestmark = pytest.mark.gpu


def _nerr(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm())


def _run(dtype, seed):
    cfg = lm_config(**TINY)
    m = init_random_(CompressedMoEModel(cfg), seed=seed)
    with torch.no_grad():
        for layer in m.layers:
            if isinstance(layer.mlp, EthosExpertLayer):
                layer.mlp.expert_latents.weight.mul_(50.0)  # expert outputs of the residual's order
    P = {k: v.detach().to(dtype).float().clone() for k, v in m.state_dict().items()}
    m = m.to(dtype).cuda().eval()
    inputs = {}
    hooks = [layer.mlp.register_forward_pre_hook(lambda mod, a, i=i: inputs.__setitem__(i, a[0].detach()))
             for i, layer in enumerate(m.layers) if isinstance(layer.mlp, EthosExpertLayer)]
    ids = torch.randint(0, cfg.vocab_size, (2, 24), generator=torch.Generator().manual_seed(seed))
    with torch.no_grad():
        logits = m(ids.cuda())
        routing = {i: m.layers[i].mlp.router(x.reshape(-1, cfg.d_model))[1].cpu() for i, x in inputs.items()}
        # the expert layers matter: without them the logits move by more than the tolerance
        base = lm_forward(P, ids, cfg, routing)
    for h in hooks:
        h.remove()
    return cfg, m, P, ids, logits, routing, base


def test_lm_forward_matches_reference_fp32():
    cfg, m, P, ids, logits, routing, ref = _run(torch.float32, 1)
    assert logits.shape == (2, 24, cfg.vocab_size) and logits.dtype == torch.float32
    assert _nerr(logits, ref) < 1e-4
    # the expert layers contribute: zeroing their v weights changes the reference logits
    P0 = dict(P)
    for i in routing:
        k = f"layers.{i}.mlp.generation_network.net.2.weight"
        w = P0[k].clone()
        w[cfg.d_model:] = 0
        P0[k] = w
    assert _nerr(lm_forward(P0, ids, cfg, routing), ref) > 1e-2


def test_lm_forward_bf16_close_to_reference():
    cfg, m, P, ids, logits, routing, ref = _run(torch.bfloat16, 2)
    assert logits.dtype == torch.bfloat16
    assert _nerr(logits.float(), ref) < 3e-2
