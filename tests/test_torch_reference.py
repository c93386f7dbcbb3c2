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
