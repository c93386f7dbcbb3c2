"""Gradients of the drop-in layer against autograd through the reference's layer
(tests/torch_reference.py restates model.py:208-254 and 288-343 in float32 on the CPU).
The reference is differentiated at the expert ids the layer chose, so both differentiate
the same selection; float32 layers must agree to 1e-4 normalised error on x and every
parameter, bf16 layers to 3e-2 against the float32 reference at the bf16-rounded values."""
import numpy as np
import pytest
import torch

import ethos_amd
from ethos_amd.workloads import SHAPES, make_inputs
from torch_reference import layer_forward, leaves

pytestmark = pytest.mark.gpu


def _nerr(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / max(float(b.norm()), 1e-30))


def _grads(name, train, signal=True, hidden=False):
    sh = SHAPES[name]
    x, sd = make_inputs(sh, signal=signal)
    m = ethos_amd.EthosExpertLayer(sh.config(), hidden_space=hidden).to(sh.torch_dtype)
    m.load_state_dict(sd)
    m = m.cuda().train(train)
    xd = x.cuda().view(sh.batch, -1, sh.d_model).clone().requires_grad_(True)
    y = m(xd)
    w = torch.randn(y.shape, generator=torch.Generator().manual_seed(1)).to(y.dtype).cuda()
    (y.float() * w.float()).sum().backward()
    with torch.no_grad():
        _, ids = m.router(xd.detach().view(-1, sh.d_model))
    # the reference at the same (dtype-rounded) values, in float32
    P = leaves({k: v.to(sh.torch_dtype) for k, v in sd.items()})
    xr = x.to(sh.torch_dtype).float().clone().requires_grad_(True)
    yr, _ = layer_forward(P, xr, sh.num_heads, sh.top_k, bn_batch_stats=train, ids=ids.cpu())
    (yr * w.float().cpu().view(yr.shape)).sum().backward()
    ours = {"x": xd.grad.view(-1, sh.d_model)}
    ours.update({k: p.grad for k, p in m.named_parameters()})
    ref = {"x": xr.grad}
    ref.update({k: P[k].grad for k, _ in m.named_parameters()})
    return sh, m, y, yr, ours, ref


@pytest.mark.parametrize("name,train,hidden", [("tiny_fp32", False, False), ("tiny_fp32", True, False),
                                               ("cfg1", False, False), ("cfg1", True, False),
                                               ("tiny_fp32", True, True), ("cfg1", False, True)])
def test_grads_match_reference_fp32(name, train, hidden):
    sh, m, y, yr, ours, ref = _grads(name, train, hidden=hidden)
    assert _nerr(y.view(-1, sh.d_model), yr) < 1e-5
    for k in ref:
        assert ours[k] is not None, k
        if train and k.startswith("router.query_projs.") and k.endswith(".bias"):
            # batch-statistics BatchNorm subtracts the batch mean, so the projection bias
            # has zero gradient: both sides hold rounding noise only
            wk = k[: -len("bias")] + "weight"
            scale = float(ref[wk].norm())
            assert float(ours[k].norm()) < 1e-5 * scale and float(ref[k].norm()) < 1e-5 * scale, k
            continue
        assert ref[k] is not None and float(ref[k].norm()) > 0, k
        e = _nerr(ours[k], ref[k])
        assert e < 1e-4, (k, e)


@pytest.mark.parametrize("train", [False, True])
def test_grads_match_reference_bf16(train):
    sh, m, y, yr, ours, ref = _grads("tiny", train)
    for k in ref:
        if train and k.startswith("router.query_projs.") and k.endswith(".bias"):
            continue  # zero gradient under batch statistics (see the fp32 test)
        e = _nerr(ours[k].float(), ref[k])
        assert e < 3e-2, (k, e)
        assert ours[k].dtype == torch.bfloat16


@pytest.mark.parametrize("name", ["cfg3", "tiny_fp32"])
def test_backward_deterministic(name):
    """Two forward + backward passes of the layer on the same input give bit-identical
    gradients for x and every parameter (the expert sums have a fixed order)."""
    sh = SHAPES[name]
    x, sd = make_inputs(sh, signal=True)
    grads = []
    for _ in range(2):
        m = ethos_amd.EthosExpertLayer(sh.config()).to(sh.torch_dtype)
        m.load_state_dict(sd)
        m = m.cuda().train()
        xd = x.cuda().view(sh.batch, -1, sh.d_model).clone().requires_grad_(True)
        y = m(xd)
        w = torch.randn(y.shape, generator=torch.Generator().manual_seed(1)).to(y.dtype).cuda()
        (y.float() * w.float()).sum().backward()
        torch.cuda.synchronize()
        grads.append({"x": xd.grad.clone(), **{k: p.grad.clone() for k, p in m.named_parameters()}})
    assert grads[0].keys() == grads[1].keys()
    for k in grads[0]:
        assert torch.equal(grads[0][k], grads[1][k]), f"{name}: gradient of {k} differs between two runs"


def test_grad_path_forward_values_unchanged():
    """Autograd on or off, the forward output is the same HIP result bit for bit, and only
    the autograd pass carries a graph; BatchNorm running stats advance once per call."""
    sh = SHAPES["tiny"]
    x, sd = make_inputs(sh, signal=True)
    m = ethos_amd.EthosExpertLayer(sh.config()).to(sh.torch_dtype)
    m.load_state_dict(sd)
    m = m.cuda().eval()
    xd = x.cuda().view(sh.batch, -1, sh.d_model)
    with torch.no_grad():
        y0 = m(xd)
    y1 = m(xd.clone().requires_grad_(True))
    assert y0.grad_fn is None and y1.grad_fn is not None
    assert torch.equal(y0, y1.detach())
    scores, ids = m.router(xd.view(-1, sh.d_model).clone().requires_grad_(True))
    with torch.no_grad():
        s0, i0 = m.router(xd.view(-1, sh.d_model))
    assert scores.grad_fn is not None and torch.equal(scores.detach(), s0) and torch.equal(ids, i0)
    m.train()
    nbt = int(m.router.query_norms[0].num_batches_tracked)
    m(xd.clone().requires_grad_(True)).sum().backward()
    assert int(m.router.query_norms[0].num_batches_tracked) == nbt + 1


def test_cfg3_backward_runs_and_matches_reference_on_experts():
    """Config 3 (64 tokens, 262,144 experts, bf16): gradients of the generator weights and
    latents against the float32 reference at the layer's ids."""
    sh = SHAPES["cfg3"]
    x, sd = make_inputs(sh, signal=True)
    m = ethos_amd.EthosExpertLayer(sh.config()).to(sh.torch_dtype)
    m.load_state_dict(sd)
    m = m.cuda().eval()
    xd = x.cuda().view(1, -1, sh.d_model).clone().requires_grad_(True)
    y = m(xd)
    (y.float() ** 2).sum().backward()
    with torch.no_grad():
        _, ids = m.router(xd.detach().view(-1, sh.d_model))
    P = leaves({k: v.to(sh.torch_dtype) for k, v in sd.items()})
    xr = x.to(sh.torch_dtype).float().clone().requires_grad_(True)
    yr, _ = layer_forward(P, xr, sh.num_heads, sh.top_k, bn_batch_stats=False, ids=ids.cpu())
    (yr ** 2).sum().backward()
    for k in ("generation_network.net.0.weight", "generation_network.net.2.weight"):
        assert _nerr(dict(m.named_parameters())[k].grad.float(), P[k].grad) < 3e-2, k
    lat = m.expert_latents.weight.grad.float().cpu()
    used = np.unique(ids.cpu().numpy())
    assert _nerr(lat[used], P["expert_latents.weight"].grad[used]) < 3e-2
    unused = np.setdiff1d(np.arange(sh.num_experts), used)[:1000]
    assert float(lat[unused].abs().max()) == 0.0
    assert _nerr(xd.grad.view(-1, sh.d_model).float(), xr.grad) < 3e-2


@pytest.mark.parametrize("dt,n,H,k,dh,E,hot", [("bf16", 50, 2, 4, 64, 37, 0.0), ("bf16", 33, 8, 16, 512, 900, 0.0),
                                               ("fp32", 20, 4, 8, 96, 11, 0.0), ("bf16", 7, 3, 5, 40, 3, 0.0),
                                               ("bf16", 300, 8, 16, 512, 5000, 0.5), ("fp32", 64, 4, 8, 128, 1, 0.0)])
def test_expert_backward_entry_point(dt, n, H, k, dh, E, hot):
    """ethos_expert_backward through the C-ABI against a float64 torch evaluation of its four
    outputs (dscores, hacc, dxp, dh), on routing sorted by ethos_sort_segment: experts with
    repeated pairs, a hot expert holding half of 38,400 pairs (a segment across ~300 blocks of
    the expert-sum pass), and one expert holding every pair.  Two runs are bit-identical."""
    from ethos_amd import hip
    g = torch.Generator().manual_seed(n + dh)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    ids = torch.randint(0, E, (n * H * k,), generator=g, dtype=torch.int32)
    if hot > 0:
        ids[torch.rand(ids.numel(), generator=g) < hot] = 7
    seg = hip.sort_segment(ids.cuda(), E)
    U = int(seg["n_unique"].item())
    slot = seg["pair_slot"].cpu()
    h = (torch.randn(U, dh, generator=g) * 0.5).to(tdt)
    xp = torch.randn(n, dh, generator=g)
    dyb = torch.randn(n, dh, generator=g)
    gates = torch.rand(n, H, k, generator=g).to(tdt)
    dg, hacc, dxp, dhs = hip.expert_backward(h.cuda(), xp.cuda(), dyb.cuda(), seg, gates.cuda(), H, k, U)
    again = hip.expert_backward(h.cuda(), xp.cuda(), dyb.cuda(), seg, gates.cuda(), H, k, U)
    torch.cuda.synchronize()
    for a1, a2, name in zip((dg, hacc, dxp, dhs), again, ("dscores", "hacc", "dxp", "dh")):
        assert torch.equal(a1, a2), f"{name} differs between two runs"
    hd, x64, y64 = h.double(), xp.double(), dyb.double()
    t = torch.arange(n * H * k) // (H * k)
    hs = hd[slot.long()]
    c = (hs * x64[t]).sum(-1)
    act = torch.nn.functional.gelu(c)
    gp = gates.double().reshape(-1)
    da = (hs * y64[t]).sum(-1)
    cdf = 0.5 * torch.erfc(-c / 2 ** 0.5)
    dgelu = cdf + c * torch.exp(-0.5 * c * c) / (2 * torch.pi) ** 0.5
    dc = gp * dgelu * da
    a = act * gp
    ref_dg = (act * da).view(n, H, k)
    ref_hacc = torch.zeros(n, dh, dtype=torch.float64).index_add_(0, t, a[:, None] * hs)
    ref_dxp = torch.zeros(n, dh, dtype=torch.float64).index_add_(0, t, dc[:, None] * hs)
    ref_dh = torch.zeros(U, dh, dtype=torch.float64).index_add_(0, slot.long(), a[:, None] * y64[t] + dc[:, None] * x64[t])
    for got, ref, name in ((dg, ref_dg, "dscores"), (hacc, ref_hacc, "hacc"), (dxp, ref_dxp, "dxp"), (dhs, ref_dh, "dh")):
        assert got.shape == ref.shape, name
        assert _nerr(got, ref) < 1e-5, (name, _nerr(got, ref))
