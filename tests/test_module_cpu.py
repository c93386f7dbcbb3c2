"""Host-side behaviour of the drop-in modules (no GPU needed)."""
import numpy as np
import pytest
import torch

import ethos_amd
from ethos_amd.workloads import SHAPES, make_inputs
from golden_util import load
from oracle import loop_faithful, oracle as O

REFERENCE_KEYS_H2 = sorted(
    ["expert_latents.weight", "generation_network.net.0.weight", "generation_network.net.2.weight",
     "router.sub_keys_1.weight", "router.sub_keys_2.weight"]
    + [f"router.query_projs.{h}.{n}" for h in range(2) for n in ("weight", "bias")]
    + [f"router.query_norms.{h}.{n}" for h in range(2)
       for n in ("weight", "bias", "running_mean", "running_var", "num_batches_tracked")]
)


def test_state_dict_keys_match_reference_layout():
    sh = SHAPES["tiny"]
    m = ethos_amd.EthosExpertLayer(sh.config())
    assert sorted(m.state_dict().keys()) == REFERENCE_KEYS_H2
    x, sd = make_inputs(sh)
    m.to(torch.bfloat16).load_state_dict(sd)  # strict
    assert m.router.num_sub_keys == 16
    assert ethos_amd.SimplifiedHypernetMoE is ethos_amd.FusedLowRankMoE_Reordered is ethos_amd.EthosExpertLayer


def test_constructor_rejects_non_square_expert_count():
    cfg = SHAPES["tiny"].config()
    cfg.num_experts = 250
    with pytest.raises(AssertionError):
        ethos_amd.EthosExpertLayer(cfg)


def test_forward_refuses_cpu_tensors():
    sh = SHAPES["tiny"]
    m = ethos_amd.EthosExpertLayer(sh.config())
    with pytest.raises(RuntimeError, match="HIP device"):
        m(torch.zeros(1, 4, sh.d_model))
    with pytest.raises(RuntimeError, match="HIP device"):
        m.router(torch.zeros(4, sh.d_model))


def test_bn_coefficients_match_oracle_bitwise():
    """The module's host-side BatchNorm coefficients equal the oracle's (both fp32 IEEE)."""
    sh = SHAPES["tiny"]
    m = ethos_amd.EthosExpertLayer(sh.config())
    g = torch.Generator().manual_seed(5)
    for bn in m.router.query_norms:
        bn.weight.data = torch.rand(sh.d_query, generator=g) + 0.5
        bn.bias.data = torch.randn(sh.d_query, generator=g)
        bn.running_mean.data = torch.randn(sh.d_query, generator=g)
        bn.running_var.data = torch.rand(sh.d_query, generator=g) + 0.1
    _, _, _, _, alpha, beta = m.router._packed(torch.float32, torch.device("cpu"))
    for h, bn in enumerate(m.router.query_norms):
        a, b = O.bn_coeffs(bn.weight.detach().numpy(), bn.bias.detach().numpy(), bn.running_mean.numpy(),
                           bn.running_var.numpy())
        assert np.array_equal(alpha[h].numpy(), a) and np.array_equal(beta[h].numpy(), b)


@pytest.mark.parametrize("name", ["tiny", "tiny_fp32", "cfg1"])
def test_loop_faithful_baseline_reproduces_reference(name):
    """The CPU baseline (a loop-faithful restatement) is bit-identical to the reference."""
    f, meta = load(name)
    sh = SHAPES[meta["shape"]]
    x, sd = make_inputs(sh, signal=meta["signal"])
    with torch.no_grad():
        gates, ids = loop_faithful.route(x, sd, sh.num_heads, sh.top_k)
        y = loop_faithful.layer(x, sd, sh.num_heads, sh.top_k)
    assert np.array_equal(ids.numpy().astype(np.int32), f["ref_indices"])
    assert np.array_equal(O.from_torch(y), f["ref_out"])
