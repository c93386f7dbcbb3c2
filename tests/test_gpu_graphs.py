"""Graph-captured layer forwards (ethos_amd.graphs.CapturedLayer): every replay equals the
eager forward bit for bit, with eager work and synchronisations between the replays, and a
parameter change leads to a new capture."""
import pytest
import torch

import ethos_amd
from ethos_amd.graphs import CapturedLayer
from ethos_amd.workloads import SHAPES, make_inputs


def _layer(sh, sd):
    m = ethos_amd.EthosExpertLayer(sh.config()).to(sh.torch_dtype)
    m.load_state_dict(sd)
    return m.cuda().eval()


def _inputs(sh, n):
    g = torch.Generator(device="cpu").manual_seed(n)
    return [torch.randn((sh.n_tok, sh.d_model), generator=g).to(sh.torch_dtype).cuda() for _ in range(n)]


@pytest.mark.gpu
@pytest.mark.parametrize("name,overlap,hidden_space", [("cfg3", True, False), ("cfg3", False, False),
                                                       ("cfg3", True, True), ("tiny_fp32", True, False),
                                                       ("cfg1", True, False)])
def test_captured_layer_replays_equal_eager(name, overlap, hidden_space):
    sh = SHAPES[name]
    _, sd = make_inputs(sh, signal=True)
    m = _layer(sh, sd)
    m.hidden_space = hidden_space
    cap = CapturedLayer(m, sh.n_tok, overlap_token_proj=overlap)
    with torch.no_grad():
        for x in _inputs(sh, 4):
            want = m.forward_flat(x)
            torch.cuda.synchronize()
            got = cap(x).clone()
            torch.cuda.synchronize()
            assert torch.equal(got, want)
            # eager work between replays, then the same input again
            m.forward_flat(x.flip(0))
            torch.cuda.synchronize()
            assert torch.equal(cap(x), want)


@pytest.mark.gpu
def test_captured_layer_recaptures_after_a_parameter_change():
    sh = SHAPES["cfg3"]
    _, sd = make_inputs(sh, signal=True)
    m = _layer(sh, sd)
    cap = CapturedLayer(m, sh.n_tok)
    x = _inputs(sh, 1)[0]
    before = cap(x).clone()
    graph = cap.graph
    with torch.no_grad():
        m.generation_network.net[2].weight.mul_(2.0)
        m.router.sub_keys_1.weight.add_(0.01)
        want = m.forward_flat(x)
    got = cap(x)
    torch.cuda.synchronize()
    assert cap.graph is not graph
    assert torch.equal(got, want) and not torch.equal(got, before)
    # a parameter replaced by a new object (no version change on the old one) is seen too
    graph = cap.graph
    lat = m.expert_latents.weight
    m.expert_latents.weight = torch.nn.Parameter(lat.detach() * 3.0)
    with torch.no_grad():
        want = m.forward_flat(x)
    got = cap(x)
    torch.cuda.synchronize()
    assert cap.graph is not graph and torch.equal(got, want)


@pytest.mark.gpu
def test_captured_layer_rejects_other_shapes():
    sh = SHAPES["tiny"]
    _, sd = make_inputs(sh)
    m = _layer(sh, sd)
    cap = CapturedLayer(m, sh.n_tok)
    with pytest.raises(RuntimeError, match="CapturedLayer takes"):
        cap(torch.zeros((sh.n_tok + 1, sh.d_model), dtype=sh.torch_dtype, device="cuda"))


def test_captured_layer_needs_eval_mode_and_a_device():
    sh = SHAPES["tiny"]
    _, sd = make_inputs(sh)
    m = ethos_amd.EthosExpertLayer(sh.config()).to(sh.torch_dtype)
    m.load_state_dict(sd)
    with pytest.raises(RuntimeError, match="eval mode"):
        CapturedLayer(m.train(), sh.n_tok)
    with pytest.raises(RuntimeError, match="HIP device"):
        CapturedLayer(m.eval(), sh.n_tok)
