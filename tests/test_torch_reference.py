"""CPU checks of the gradient references: the float32 torch restatement of the reference
layer (tests/torch_reference.py) against the oracle's forward, and the GELU derivative the
layer's backward uses against autograd."""
import numpy as np
import torch

from ethos_amd.layer import _gelu_grad
from ethos_amd.workloads import SHAPES, make_inputs
from oracle import oracle as O
from torch_reference import layer_forward, leaves


def test_gelu_grad_matches_autograd():
    x = torch.linspace(-12, 12, 20001, dtype=torch.float64, requires_grad=True)
    torch.nn.functional.gelu(x).sum().backward()
    assert torch.allclose(_gelu_grad(x.detach()), x.grad, rtol=1e-12, atol=1e-14)


def test_torch_reference_forward_matches_oracle():
    """Same routing (ids, checked equal) and the same outputs as the oracle's fp32 layer, with
    the routing chosen by the restatement's own topk and then imposed again through `ids`."""
    sh = SHAPES["tiny_fp32"]
    x, sd = make_inputs(sh, signal=True)
    P = leaves(sd)
    with torch.no_grad():
        y, ids = layer_forward(P, x.float(), sh.num_heads, sh.top_k, bn_batch_stats=False)
        y2, _ = layer_forward(P, x.float(), sh.num_heads, sh.top_k, bn_batch_stats=False, ids=ids)
    Po = O.unpack_state(sd, sh.num_heads)
    r = O.layer_forward(O.from_torch(x), Po, sh.num_heads, sh.top_k, "fp32")
    assert np.array_equal(ids.numpy(), r["ids"])
    ref = r["out"].astype(np.float64)
    for out in (y, y2):
        d = np.abs(out.numpy().astype(np.float64) - ref)
        assert d.max() <= 1e-5 * np.abs(ref).max(), d.max()


def test_apply_from_routing_matches_oracle():
    """The float32 expert stages for an imposed routing (the oracle's ids and gates) against
    the oracle's fp32 layer output, and a dropped pair or a wrong slot shows up far above the
    agreement on every token it touches."""
    from torch_reference import apply_from_routing

    sh = SHAPES["tiny_fp32"]
    x, sd = make_inputs(sh, signal=True)
    Po = O.unpack_state(sd, sh.num_heads)
    r = O.layer_forward(O.from_torch(x), Po, sh.num_heads, sh.top_k, "fp32")
    gates, ids = torch.from_numpy(np.asarray(r["gates"], np.float32)), torch.from_numpy(r["ids"])
    with torch.no_grad():
        y, scale = apply_from_routing(sd, x.float(), gates, ids, sh.num_heads, chunk=5)
    ref = torch.from_numpy(r["out"].astype(np.float32))
    # (a token whose activations all underflow has scale 0: measured against 1e-3 of the largest)
    scale = scale.clamp_min(1e-3 * float(scale.max()))
    err = (y - ref).norm(dim=1) / scale
    assert float(err.max()) < 1e-4, float(err.max())
    # a dropped pair (gate zeroed) and a pair moved to another expert, on token 3
    g2 = gates.clone()
    g2[3, 0, 2] = 0.0
    ids2 = ids.clone()
    ids2[3, 1, 0] = (ids2[3, 1, 0] + 1) % sd["expert_latents.weight"].shape[0]
    for g, i in ((g2, ids), (gates, ids2)):
        with torch.no_grad():
            y2, _ = apply_from_routing(sd, x.float(), g, i, sh.num_heads)
        e2 = (y2 - ref).norm(dim=1) / scale
        assert float(e2[3]) > 1e-2 and float(torch.cat([e2[:3], e2[4:]]).max()) < 1e-4
