"""The drop-in layer (ethos_amd.EthosExpertLayer) on the GPU against the oracle and
against the reference's own outputs (tests/golden)."""
import numpy as np
import pytest
import torch

import ethos_amd
from ethos_amd import hip
from ethos_amd.workloads import SHAPES, make_inputs
from golden_util import load
from gpu_util import check_all_tokens, check_out, to_dev, to_host
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _layer(sh, sd):
    m = ethos_amd.EthosExpertLayer(sh.config()).to(sh.torch_dtype)
    m.load_state_dict(sd)
    return m.cuda().eval()


@pytest.mark.parametrize("name,signal", [("tiny", False), ("tiny", True), ("tiny_fp32", False), ("tiny_fp32", True),
                                         ("cfg1", False), ("cfg1", True), ("cfg1_dq128", False), ("cfg3", False),
                                         ("cfg3", True)])
def test_layer_matches_oracle(name, signal):
    sh = SHAPES[name]
    x, sd = make_inputs(sh, signal=signal)
    m = _layer(sh, sd)
    xd = x.cuda().view(sh.batch, sh.n_tok // sh.batch, sh.d_model)
    with torch.no_grad():
        gates, ids = m.router(xd.view(-1, sh.d_model))
        y = m(xd)
    torch.cuda.synchronize()
    P = O.unpack_state(sd, sh.num_heads)
    r = O.layer_forward(O.from_torch(x), P, sh.num_heads, sh.top_k, sh.dtype)
    assert ids.dtype == torch.int64 and ids.shape == (sh.n_tok, sh.num_heads, sh.top_k)
    assert np.array_equal(ids.cpu().numpy(), r["ids"]), "routing indices differ from the oracle"
    assert np.array_equal(O.to_f32(to_host(gates), sh.dtype), O.to_f32(r["gates"], sh.dtype)) or sh.dtype == "fp32"
    assert y.shape == xd.shape and y.dtype == xd.dtype
    check_out(O.to_f32(to_host(y.reshape(sh.n_tok, -1)), sh.dtype), r["out"], sh.dtype, signal=signal,
              nerr_max=2e-3)


@pytest.mark.parametrize("name", ["tiny", "tiny_signal", "tiny_fp32", "tiny_fp32_signal", "cfg1", "cfg1_signal",
                                  "cfg1_dq128", "cfg3", "cfg3_signal"])
def test_layer_against_reference_outputs(name):
    """Reference fixtures: fp32 routing identical and outputs within rtol 1e-4; bf16
    routing equal up to the reference's arbitrary tie choices (same combined-score
    values), and the expert stage fed the reference's routing within the bf16 bar."""
    f, meta = load(name)
    sh = SHAPES[meta["shape"]]
    x, sd = make_inputs(sh, signal=meta["signal"])
    m = _layer(sh, sd)
    xd = x.cuda()
    with torch.no_grad():
        gates, ids = m.router(xd)
        y = m(xd.view(1, sh.n_tok, sh.d_model)).view(sh.n_tok, -1)
    ref_ids = f["ref_indices"]
    if sh.dtype == "fp32":
        assert np.array_equal(ids.cpu().numpy(), ref_ids)
        check_out(y.cpu().numpy(), f["ref_out"], "fp32")
    else:
        # same multiset of gate values in every row (the gates are a function of the
        # combined scores), i.e. any difference is a choice inside a tied group
        theirs = np.sort(O.to_f32(f["ref_scores"], "bf16"), -1)
        # 1. routing of the reference's own queries: every (token, head) row selects the
        #    same multiset of gates as the reference (ids can differ only inside tied
        #    groups, which torch.topk breaks arbitrarily)
        rq = to_dev(f["ref_q"])
        g_rq, _ = hip.route_topk(rq, m.router.sub_keys_1.weight.detach(), m.router.sub_keys_2.weight.detach(),
                                 sh.top_k)
        rows_rq = int(np.any(np.sort(O.to_f32(to_host(g_rq), "bf16"), -1) != theirs, -1).sum())
        print(f"{name}: routing the reference's queries, {rows_rq} of {theirs.shape[0] * theirs.shape[1]} rows "
              "with differing gate multisets")
        assert rows_rq == 0, rows_rq
        # 2. routing from x: the layer's queries are the correctly rounded projection, the
        #    reference's are torch's bf16 GEMM; a row may differ only where those differ
        ours = np.sort(O.to_f32(to_host(gates), "bf16"), -1)
        rows = np.any(ours != theirs, -1)
        q_rows = np.any(to_host(m.router.queries(xd)) != f["ref_q"], -1)
        print(f"{name}: routing from x, {int(rows.sum())} rows with differing gate multisets, all among the "
              f"{int(q_rows.sum())} rows whose reference query differs from the correctly rounded one")
        assert not np.any(rows & ~q_rows)
        # expert stage with the reference's routing
        seg = hip.sort_segment(to_dev(ref_ids.reshape(-1).astype(np.int32)), sh.num_experts)
        w2 = m.generation_network.net[2].weight.detach()
        h, v = hip.generate(m.expert_latents.weight.detach(), seg["uniq"], seg["n_unique"], seg["max_unique"],
                            m.generation_network.net[0].weight.detach(), w2)
        out = hip.apply_scatter(xd, w2, h, v, seg, to_dev(f["ref_scores"]), sh.num_heads, sh.top_k)
        check_out(O.to_f32(to_host(out), "bf16"), O.to_f32(f["ref_out"], "bf16"), "bf16", signal=meta["signal"])


def test_layer_deterministic():
    sh = SHAPES["cfg3"]
    x, sd = make_inputs(sh)
    m = _layer(sh, sd)
    xd = x.cuda().view(1, sh.n_tok, -1)
    with torch.no_grad():
        a = m(xd).clone()
        b = m(xd).clone()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_layer_linear_in_v():
    """Doubling the v half of the generator's output layer doubles the output exactly."""
    sh = SHAPES["cfg3"]
    x, sd = make_inputs(sh, signal=True)
    m = _layer(sh, sd)
    xd = x.cuda().view(1, sh.n_tok, -1)
    with torch.no_grad():
        y1 = m(xd).float()
        m.generation_network.net[2].weight[sh.d_model:] *= 2
        y2 = m(xd).float()
    assert torch.equal(y2, 2 * y1)


def test_layer_cfg2_full_size():
    """Config 2 at full size: the queries of all 4,096 tokens and every routing row (ids
    and gates) bit-exact against the oracle, sort invariants on all pairs, and the
    output of 512 tokens (every 8th) against the oracle."""
    sh = SHAPES["cfg2"]
    x, sd = make_inputs(sh)
    m = _layer(sh, sd)
    xd = x.cuda()
    with torch.no_grad():
        q = m.router.queries(xd)
        gates, ids = m.router.route(xd)
        seg = hip.sort_segment(ids.view(-1), sh.num_experts)
        y = m(xd.view(sh.batch, -1, sh.d_model)).view(sh.n_tok, -1)
    torch.cuda.synchronize()
    P = O.unpack_state(sd, sh.num_heads)
    xs = O.from_torch(x)
    q_ref = O.query_proj(xs, P["Wq"], P["bq"], P["alpha"], P["beta"], "bf16")
    qh = to_host(q)
    print(f"cfg2: {int(np.count_nonzero(qh != q_ref))} of {qh.size} query elements differ from the oracle")
    assert np.array_equal(qh, q_ref)
    g_ref, ids_ref = O.route(qh, P["K1"], P["K2"], sh.top_k, "bf16")
    ih, gh = to_host(ids), to_host(gates)
    print(f"cfg2: {int(np.any(ih != ids_ref, -1).sum())} routing rows with differing ids, "
          f"{int(np.count_nonzero(gh != g_ref))} differing gates")
    assert np.array_equal(ih, ids_ref)
    assert np.array_equal(gh, g_ref)
    # sort invariants on the full pair set
    flat = ids.view(-1).long()
    perm = seg["perm"].long()
    U = int(seg["n_unique"].item())
    assert torch.equal(torch.sort(perm).values, torch.arange(flat.numel(), device="cuda"))
    ks = flat[perm]
    assert bool((ks[1:] >= ks[:-1]).all())
    uq = torch.unique(flat)
    assert U == uq.numel() and torch.equal(seg["uniq"][:U].long(), uq)
    # output for 512 tokens
    sub = np.arange(0, sh.n_tok, 8)
    r = O.layer_forward(xs, P, sh.num_heads, sh.top_k, "bf16", tokens=sub, q=qh)
    check_out(O.to_f32(to_host(y), "bf16")[sub], r["out"], "bf16", nerr_max=2e-3)
    check_all_tokens(m, xd, gates, ids, y, "cfg2")


def test_layer_cfg4_zipf_full_size():
    """Config 4 at full size: 32,768 tokens with Zipf(1.1)-skewed sub-key rows, so a few
    thousand unique experts carry 4.2 M pairs and the largest segments hold tens of
    thousands of pairs.  Every routing row (ids and gates) bit-exact against the oracle,
    segment offsets against a histogram of the ids, and the output of a token subset
    against the oracle."""
    sh = SHAPES["cfg4"]
    x, sd = make_inputs(sh)
    m = _layer(sh, sd)
    xd = x.cuda()
    with torch.no_grad():
        q = m.router.queries(xd)
        gates, ids = m.router.route(xd)
        seg = hip.sort_segment(ids.view(-1), sh.num_experts)
        y = m(xd.view(sh.batch, -1, sh.d_model)).view(sh.n_tok, -1)
    torch.cuda.synchronize()
    P = O.unpack_state(sd, sh.num_heads)
    xs = O.from_torch(x)
    qh = to_host(q)
    sub = np.arange(0, sh.n_tok, 16)
    # the query projection on every 4th token (8,192 tokens, 16.8 M outputs)
    qsub = np.arange(0, sh.n_tok, 4)
    q_ref = O.query_proj(xs[qsub], P["Wq"], P["bq"], P["alpha"], P["beta"], "bf16")
    assert np.array_equal(qh[qsub], q_ref)
    g_ref, ids_ref = O.route(qh, P["K1"], P["K2"], sh.top_k, "bf16")
    assert np.array_equal(to_host(ids), ids_ref)
    gh = to_host(gates)
    print(f"cfg4: {int(np.count_nonzero(gh != g_ref))} of {gh.size} gates differ from the oracle")
    assert np.array_equal(gh, g_ref)
    # segments: unique ids ascending, offsets = running histogram of the ids
    flat = ids.view(-1).long()
    U = int(seg["n_unique"].item())
    uq, counts = torch.unique(flat, return_counts=True)
    assert U == uq.numel() and torch.equal(seg["uniq"][:U].long(), uq)
    off = seg["seg_off"][: U + 1].long()
    assert int(off[0]) == 0 and torch.equal(off[1:] - off[:-1], counts)
    assert int(counts.max()) > 10_000, "the skew should give segments of tens of thousands of pairs"
    perm = seg["perm"].long()
    assert torch.equal(torch.sort(perm).values, torch.arange(flat.numel(), device="cuda"))
    assert bool((flat[perm][1:] >= flat[perm][:-1]).all())
    # output for a token subset (every 16th token: 2,048)
    r = O.layer_forward(xs, P, sh.num_heads, sh.top_k, "bf16", tokens=sub, q=qh)
    check_out(O.to_f32(to_host(y), "bf16")[sub], r["out"], "bf16", nerr_max=2e-3)
    check_all_tokens(m, xd, gates, ids, y, "cfg4")


def test_router_rejects_cpu_and_bad_shapes():
    sh = SHAPES["tiny"]
    x, sd = make_inputs(sh)
    m = _layer(sh, sd)
    with pytest.raises(RuntimeError):
        m(x.view(1, sh.n_tok, -1))  # CPU input: no CPU path
    wide = torch.zeros((1, sh.n_tok, 2 * sh.d_model), dtype=sh.torch_dtype, device="cuda")
    with pytest.raises(RuntimeError, match="contiguous"):
        m(wide[:, :, : sh.d_model])  # a non-viewable input, as x.view(-1, d) would reject
    with pytest.raises(RuntimeError):
        m(x.cuda())  # not [batch, seq, d_model]


def test_empty_input():
    sh = SHAPES["tiny"]
    x, sd = make_inputs(sh)
    m = _layer(sh, sd)
    y = m(torch.empty((0, 5, sh.d_model), dtype=sh.torch_dtype, device="cuda"))
    assert y.shape == (0, 5, sh.d_model)


@pytest.mark.parametrize("name,signal", [("tiny", True), ("tiny_fp32", True), ("cfg1", False), ("cfg3", False),
                                         ("cfg3", True)])
def test_layer_hidden_space(name, signal):
    """The layer with hidden_space=True: the same routing as the default layer, the output
    against the oracle's whole layer (reference algorithm) at the layer tolerance, and the
    autograd-free output of the default layer within it."""
    sh = SHAPES[name]
    x, sd = make_inputs(sh, signal=signal)
    m = _layer(sh, sd)
    mh = ethos_amd.EthosExpertLayer(sh.config(), hidden_space=True).to(sh.torch_dtype)
    mh.load_state_dict(sd)
    mh = mh.cuda().eval()
    xd = x.cuda().view(sh.batch, -1, sh.d_model)
    with torch.no_grad():
        y = m(xd).view(sh.n_tok, -1)
        yh = mh(xd).view(sh.n_tok, -1)
    torch.cuda.synchronize()
    P = O.unpack_state(sd, sh.num_heads)
    r = O.layer_forward(O.from_torch(x), P, sh.num_heads, sh.top_k, sh.dtype)
    got = O.to_f32(to_host(yh), sh.dtype)
    check_out(got, r["out"], sh.dtype, signal=signal, nerr_max=1e-2)
    check_out(got, O.to_f32(to_host(y), sh.dtype), sh.dtype, signal=signal, nerr_max=1e-2)


def test_layer_hidden_space_cfg2_subset():
    """Config 2 in hidden-space order: a token subset against the oracle's reference-algorithm
    layer and its Algorithm-1 form."""
    sh = SHAPES["cfg2"]
    x, sd = make_inputs(sh)
    mh = ethos_amd.EthosExpertLayer(sh.config(), hidden_space=True).to(sh.torch_dtype)
    mh.load_state_dict(sd)
    mh = mh.cuda().eval()
    xd = x.cuda()
    with torch.no_grad():
        q = mh.router.queries(xd)
        y = mh(xd.view(sh.batch, -1, sh.d_model)).view(sh.n_tok, -1)
    torch.cuda.synchronize()
    P = O.unpack_state(sd, sh.num_heads)
    xs = O.from_torch(x)
    sub = np.arange(0, sh.n_tok, 64)
    r = O.layer_forward(xs, P, sh.num_heads, sh.top_k, "bf16", tokens=sub, q=to_host(q))
    check_out(O.to_f32(to_host(y), "bf16")[sub], r["out"], "bf16", nerr_max=1e-2)


def test_library_stream_is_torch_current_stream():
    """The stream handed to the library is torch's current stream, also inside a stream
    context (the raw accessor the wrappers use agrees with torch.cuda.current_stream)."""
    assert hip._stream() == torch.cuda.current_stream().cuda_stream
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        assert hip._stream() == s.cuda_stream == torch.cuda.current_stream().cuda_stream
    assert hip._stream() == torch.cuda.current_stream().cuda_stream
