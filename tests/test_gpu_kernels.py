"""Each HIP stage against the oracle on identical inputs (through the C-ABI).

Bars: query projection, sub-key routing ids, the sort and the segmentation are
bit-exact; gates bit-exact in bf16 and fp32 (the softmax's exponential is the fp64 exp
rounded once to fp32 on both sides); generated expert rows and layer outputs within the stated tolerances.
"""
import numpy as np
import pytest
import torch

from ethos_amd import hip
from ethos_amd.workloads import SHAPES, make_inputs
from gpu_util import check_out, to_dev, to_host
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SMALL = ["tiny", "tiny_fp32", "cfg1", "cfg1_dq128"]


def _setup(name, n_tok=None, signal=False):
    sh = SHAPES[name]
    if n_tok is not None:
        sh = sh.with_tokens(n_tok)
    x, sd = make_inputs(sh, signal=signal)
    P = O.unpack_state(sd, sh.num_heads)
    return sh, O.from_torch(x), P


@pytest.mark.parametrize("name", SMALL + ["cfg3"])
def test_query_proj_bit_exact(name):
    sh, x, P = _setup(name)
    q_ref = O.query_proj(x, P["Wq"], P["bq"], P["alpha"], P["beta"], sh.dtype)
    q = hip.query_proj(to_dev(x), to_dev(P["Wq"]), to_dev(P["bq"]), to_dev(P["alpha"]), to_dev(P["beta"]))
    torch.cuda.synchronize()
    assert np.array_equal(to_host(q), q_ref)


@pytest.mark.parametrize("name", SMALL + ["cfg3"])
def test_query_proj_prepared_weights_bit_exact(name):
    """Weights prepared once (digit planes for bf16; nothing for fp32) and reused by two
    projections of different batches: both equal the oracle bit for bit."""
    sh, x, P = _setup(name)
    wq, bq, a, b = (to_dev(P[k]) for k in ("Wq", "bq", "alpha", "beta"))
    prep = hip.query_proj_prepare(wq)
    assert (prep is None) == (sh.dtype == "fp32")
    for rows in (slice(None), slice(0, max(1, x.shape[0] // 3))):
        xs = np.ascontiguousarray(x[rows])
        q = hip.query_proj(to_dev(xs), wq, bq, a, b, prepared=prep)
        torch.cuda.synchronize()
        assert np.array_equal(to_host(q), O.query_proj(xs, P["Wq"], P["bq"], P["alpha"], P["beta"], sh.dtype))


@pytest.mark.parametrize("name", SMALL + ["cfg3", "yaml"])
def test_route_bit_exact(name):
    sh, x, P = _setup(name)
    q = O.query_proj(x, P["Wq"], P["bq"], P["alpha"], P["beta"], sh.dtype)
    g_ref, ids_ref = O.route(q, P["K1"], P["K2"], sh.top_k, sh.dtype)
    g, ids = hip.route_topk(to_dev(q), to_dev(P["K1"]), to_dev(P["K2"]), sh.top_k)
    torch.cuda.synchronize()
    ids = to_host(ids)
    assert np.array_equal(ids, ids_ref), f"{np.sum(np.any(ids != ids_ref, -1))} rows differ"
    assert np.array_equal(O.to_f32(to_host(g), sh.dtype), O.to_f32(g_ref, sh.dtype))


@pytest.mark.parametrize("dt", ["bf16", "fp32"])
@pytest.mark.parametrize("rows", [1, 17, 80, 95, 200, 4096, 4097, 4123])
def test_route_partial_tiles_bit_exact(rows, dt):
    """Row counts that leave the last workgroup partly empty, for both row layouts (up to
    4096 rows: one row per wave, 8 per workgroup; above: four per wave, 32 per workgroup,
    with one wave holding live and dead rows and whole waves of dead rows): a regression
    test for per-row counters that were left unset past the last row."""
    rng = np.random.default_rng(rows)
    K, dh2, top_k = 16 if rows < 100 else 512, 16 if rows < 100 else 128, 4 if rows < 100 else 16
    q, k1, k2 = _stress_case("zipf", rng, rows, K, dh2, dt)
    g_ref, ids_ref = O.route(q, k1, k2, top_k, dt)
    g, ids = hip.route_topk(to_dev(q), to_dev(k1), to_dev(k2), top_k)
    torch.cuda.synchronize()
    assert np.array_equal(to_host(ids), ids_ref)
    assert np.array_equal(O.to_f32(to_host(g), dt), O.to_f32(g_ref, dt))


@pytest.mark.parametrize("dt", ["bf16", "fp32"])
@pytest.mark.parametrize("rows,K,dh2", [(200, 512, 128), (4123, 512, 128), (300, 200, 32), (5000, 100, 64),
                                        (64, 16, 16)])
def test_route_prepared_keys_bit_exact(rows, K, dh2, dt):
    """Routing with the sub-keys in fragment order (ethos_route_topk_prepared) equals the
    oracle and the unprepared call bit for bit, for both row layouts, key counts that are
    not a multiple of the 32-key blocks, and several query widths."""
    rng = np.random.default_rng(rows + K)
    top_k = 16 if K >= 32 else 4
    q, k1, k2 = _stress_case("zipf", rng, rows, K, dh2, dt)
    g_ref, ids_ref = O.route(q, k1, k2, top_k, dt)
    d1, d2 = to_dev(k1), to_dev(k2)
    prep = hip.route_prepare_keys(d1, d2)
    kn = hip.key_norm_bounds(d1, d2).cuda()
    g, ids = hip.route_topk(to_dev(q), d1, d2, top_k, key_norms=kn, prepared_keys=prep)
    g0, ids0 = hip.route_topk(to_dev(q), d1, d2, top_k, key_norms=kn)
    torch.cuda.synchronize()
    assert np.array_equal(to_host(ids), ids_ref) and torch.equal(ids, ids0)
    assert np.array_equal(O.to_f32(to_host(g), dt), O.to_f32(g_ref, dt)) and torch.equal(g, g0)


def test_route_ties_break_to_lowest_index():
    """Duplicate sub-key rows force exact score ties in both halves."""
    sh, x, P = _setup("tiny")
    K1 = P["K1"].copy()
    K2 = P["K2"].copy()
    K1[1::2] = K1[0::2]
    K2[3] = K2[5]
    q = O.query_proj(x, P["Wq"], P["bq"], P["alpha"], P["beta"], sh.dtype)
    g_ref, ids_ref = O.route(q, K1, K2, sh.top_k, sh.dtype)
    g, ids = hip.route_topk(to_dev(q), to_dev(K1), to_dev(K2), sh.top_k)
    assert np.array_equal(to_host(ids), ids_ref)


@pytest.mark.parametrize("n,E,pattern", [(1, 1, "rand"), (5, 262144, "rand"), (4096, 4096, "rand"),
                                         (8192, 4096, "rand"), (70000, 262144, "rand"), (524288, 262144, "rand"),
                                         (30000, 262144, "same"), (50000, 262144, "skew"), (4097, 7, "rand"),
                                         (12345, 262144, "max"), (300000, 262144, "rand"),
                                         (2000003, 262144, "rand"), (16384, 262144, "skew"),
                                         (16385, 262144, "skew"), (16384, 7, "rand"), (2, 262144, "same"),
                                         (8192, 262144, "max"), (70000, 7, "rand"), (100000, 4096, "rand"),
                                         (60000, 2 ** 21, "rand"), (300000, 262144, "hot2d"),
                                         (65536, 262144, "same"), (24577, 262144, "rand"),
                                         (300000, 2 ** 21, "same"), (300000, 2 ** 21, "skew"),
                                         (300000, 2 ** 21, "hot3d"), (2 ** 20, 262144, "same"),
                                         (2 ** 20 + 1, 262144, "same"), (2 ** 21 + 7, 262144, "hot2d"),
                                         (2 ** 20 + 3, 7, "rand"), (2 ** 20 + 5, 2 ** 21, "skew"),
                                         (4096 * 1024 + 4097, 262144, "rand"), (4096 * 1024 + 4097, 262144, "skew")])
def test_sort_segment_exact(n, E, pattern):
    """The sort against the oracle's counting sort: one pass (E = 7), two (4,096 and 262,144
    experts) and three (2^21) over tiles of 4,096 pairs; batches up to 16,384 pairs take the
    single-workgroup sort, batches above 2^20 pairs with ids of at most 18 bits the
    expert -> slot table for pair_slot.  Patterns: uniform ids, one id everywhere (one segment spanning
    every tile), Zipf-skewed ids, half the pairs on the largest id, and ids whose two
    9-bit digits (or, with 2^21 experts, all three digits) are Zipf-skewed (hot experts
    whose segments cross tile boundaries, in the three-pass path too).  Above 1,024 tiles the
    per-digit scans over the tiles take more than one round."""
    rng = np.random.default_rng(n + E)
    if pattern == "hot3d":
        a = np.minimum(rng.zipf(1.1, n), 512) - 1
        b = np.minimum(rng.zipf(1.1, n), 512) - 1
        c = np.minimum(rng.zipf(1.1, n), 8) - 1
        ids = ((c << 18) | (b << 9) | a).astype(np.int32)
    elif pattern == "hot2d":
        a = np.minimum(rng.zipf(1.1, n), 192) - 1
        b = np.minimum(rng.zipf(1.1, n), 192) - 1
        ids = (a * 512 + b).astype(np.int32)
    elif pattern == "same":
        ids = np.full(n, 12345, np.int32)
    elif pattern == "skew":
        ids = np.minimum((rng.zipf(1.3, n) - 1), E - 1).astype(np.int32)
    elif pattern == "max":
        ids = np.where(rng.random(n) < 0.5, E - 1, rng.integers(0, E, n)).astype(np.int32)
    else:
        ids = rng.integers(0, E, n).astype(np.int32)
    perm, uniq, seg, inv = O.sort_segment(ids, E)
    r = hip.sort_segment(to_dev(ids), E)
    torch.cuda.synchronize()
    U = int(r["n_unique"].item())
    assert U == len(uniq)
    assert np.array_equal(to_host(r["perm"]), perm)
    assert np.array_equal(to_host(r["uniq"])[:U], uniq)
    assert np.array_equal(to_host(r["seg_off"])[: U + 1], seg)
    assert np.array_equal(to_host(r["pair_slot"]), inv)
    assert np.array_equal(to_host(r["sorted_slot"]), inv[perm])


def _check_rows(got, ref, dt):
    """Generated rows against the oracle: fp32 to 1e-4; bf16 mostly identical, the rest
    one or two roundings apart (the GPU accumulates in fp32, the oracle rounds exact sums)."""
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    d = np.abs(got - ref)
    scale = np.abs(ref).max()
    if dt == "fp32":
        assert np.all(d <= 1e-4 * np.abs(ref) + 1e-5 * scale), d.max()
    else:
        ulp = np.abs(ref) * 2.0 ** -7 + 1e-30
        assert np.mean(d > 0) < 0.05, np.mean(d > 0)
        assert np.all(d <= 2 * ulp + 1e-3 * scale)
        assert np.linalg.norm(d) / np.linalg.norm(ref) < 2e-3


def _generate(lat, uniq, w1, w2, max_unique, dt):
    n_unique = torch.tensor([len(uniq)], dtype=torch.int32, device="cuda")
    h, v = hip.generate(to_dev(lat), to_dev(uniq), n_unique, max_unique, to_dev(w1), to_dev(w2))
    torch.cuda.synchronize()
    return O.to_f32(to_host(h), dt), O.to_f32(to_host(v), dt)


@pytest.mark.parametrize("name,signal", [("tiny", False), ("tiny", True), ("tiny_fp32", True), ("cfg1", True),
                                         ("cfg3", False), ("cfg3", True)])
def test_generate_matches_oracle(name, signal):
    sh, x, P = _setup(name, signal=signal)
    rng = np.random.default_rng(0)
    U = min(sh.num_experts, 777)
    uniq = np.sort(rng.choice(sh.num_experts, U, replace=False)).astype(np.int32)
    h_ref, v_ref = O.generate(P["latents"], uniq, P["W1"], P["W2"], sh.dtype)
    h, v = _generate(P["latents"], uniq, P["W1"], P["W2"], U + 5, sh.dtype)
    _check_rows(h[:U], h_ref, sh.dtype)
    _check_rows(v[:U], v_ref, sh.dtype)


def test_generate_gelu_every_bf16_input():
    """Every finite bf16 value as a pre-activation, through the generator: expert u has the
    one-hot latent e_(u % 128) and W1[j, k] is value 512 k + j, so pre = W1[j, u] exactly
    and h[u, j] must be the oracle's RN(GELU(value)) bit for bit."""
    dl, dh, d, U = 128, 512, 64, 128
    vals = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = (vals & 0x7F80) != 0x7F80
    vals = np.where(finite, vals, 0).astype(np.uint16)
    w1 = np.ascontiguousarray(vals.reshape(dl, dh).T)              # W1[j, k] = vals[512 k + j]
    lat = np.zeros((U, dl), np.uint16)
    lat[np.arange(U), np.arange(U) % dl] = O.f32_to_bf16_bits(np.ones(1, np.float32))[0]
    w2 = O.f32_to_bf16_bits(np.full((2 * d, dh), 1e-3, np.float32))
    uniq = np.arange(U, dtype=np.int32)
    h, _ = _generate(lat, uniq, w1, w2, U, "bf16")
    ref, _ = O.generate(lat, uniq, w1, w2, "bf16")
    got_bits = O.f32_to_bf16_bits(h[:U].astype(np.float32))
    ref_bits = O.f32_to_bf16_bits(ref.astype(np.float32))
    assert np.array_equal(got_bits, ref_bits), int(np.sum(got_bits != ref_bits))


@pytest.mark.parametrize("name,signal", [("tiny", False), ("tiny", True), ("tiny_fp32", True), ("cfg1", False),
                                         ("cfg3", True)])
def test_apply_matches_oracle(name, signal):
    """Given identical routing and generated rows, the scatter-back matches the oracle."""
    sh, x, P = _setup(name, signal=signal)
    q = O.query_proj(x, P["Wq"], P["bq"], P["alpha"], P["beta"], sh.dtype)
    g, ids = O.route(q, P["K1"], P["K2"], sh.top_k, sh.dtype)
    seg = hip.sort_segment(to_dev(ids.reshape(-1)), sh.num_experts)
    U = int(seg["n_unique"].item())
    w2 = to_dev(P["W2"])
    h_dev, v_dev = hip.generate(to_dev(P["latents"]), seg["uniq"], seg["n_unique"], seg["max_unique"],
                                to_dev(P["W1"]), w2)
    out = hip.apply_scatter(to_dev(x), w2, h_dev, v_dev, seg, to_dev(g), sh.num_heads, sh.top_k)
    torch.cuda.synchronize()
    h = O.to_f32(to_host(h_dev), sh.dtype)[:U]
    v = O.to_f32(to_host(v_dev), sh.dtype)[:U]
    xp = O.token_proj(x, P["W2"], sh.dtype)
    ref = O.apply(xp, h, v, to_host(seg["pair_slot"]), g, sh.num_heads, sh.top_k, sh.dtype)
    got = O.to_f32(to_host(out), sh.dtype)
    check_out(got, ref, sh.dtype, signal=signal, nerr_max=2e-3)


@pytest.mark.parametrize("n_tok,d,dh,dt", [(100, 1024, 512, "bf16"), (37, 256, 128, "bf16"), (70, 96, 64, "bf16"),
                                           (33, 128, 96, "fp32")])
def test_apply_shapes(n_tok, d, dh, dt):
    """Apply over shapes the configs do not hit: token counts that are not a multiple of
    the projection tile, widths that take the generic projection, random experts."""
    rng = np.random.default_rng(n_tok + d + dh)
    H, k, E = 2, 4, 300
    enc = (lambda a: O.f32_to_bf16_bits(a)) if dt == "bf16" else (lambda a: a.astype(np.float32))
    x = enc(rng.standard_normal((n_tok, d)).astype(np.float32))
    w2 = enc((rng.uniform(-1, 1, (2 * d, dh)) * 4 / np.sqrt(d)).astype(np.float32))
    ids = rng.integers(0, E, (n_tok, H, k)).astype(np.int32)
    g = enc(rng.uniform(0, 1, (n_tok, H, k)).astype(np.float32))
    seg = hip.sort_segment(to_dev(ids.reshape(-1)), E)
    U = int(seg["n_unique"].item())
    h = enc(rng.standard_normal((seg["max_unique"], dh)).astype(np.float32) * 0.3)
    v = enc(rng.standard_normal((seg["max_unique"], d)).astype(np.float32))
    out = hip.apply_scatter(to_dev(x), to_dev(w2), to_dev(h), to_dev(v), seg, to_dev(g), H, k)
    torch.cuda.synchronize()
    xp = O.token_proj(x, w2, dt)
    ref = O.apply(xp, O.to_f32(h, dt)[:U], O.to_f32(v, dt)[:U], to_host(seg["pair_slot"]), g, H, k, dt)
    got = O.to_f32(to_host(out), dt)
    check_out(got, ref, dt, signal=True, nerr_max=2e-3)


@pytest.mark.parametrize("n_tok,dt", [(1100, "bf16"), (40, "bf16"), (1100, "fp32")])
def test_apply_long_pair_lists(n_tok, dt):
    """More than 64 pairs per (token, head) and per token: the gathers take a head's or a
    token's pairs in chunks of 64, the next chunk loaded while one is summed, so a head's
    second chunk and the next head's first must follow in order.  Both orders of the apply,
    above 1,024 tokens (one wave per token) and below (one workgroup per token), against
    the oracle."""
    rng = np.random.default_rng(n_tok + 7)
    d, dh, H, k, E = 256, 128, 2, 70, 5000
    enc = (lambda a: O.f32_to_bf16_bits(a)) if dt == "bf16" else (lambda a: a.astype(np.float32))
    x = enc(rng.standard_normal((n_tok, d)).astype(np.float32))
    w2 = enc((rng.uniform(-1, 1, (2 * d, dh)) * 4 / np.sqrt(d)).astype(np.float32))
    ids = rng.integers(0, E, (n_tok, H, k)).astype(np.int32)
    g = enc(rng.uniform(0, 1, (n_tok, H, k)).astype(np.float32))
    seg = hip.sort_segment(to_dev(ids.reshape(-1)), E)
    U = int(seg["n_unique"].item())
    h = enc(rng.standard_normal((seg["max_unique"], dh)).astype(np.float32) * 0.3)
    v = enc(rng.standard_normal((seg["max_unique"], d)).astype(np.float32))
    out = hip.apply_scatter(to_dev(x), to_dev(w2), to_dev(h), to_dev(v), seg, to_dev(g), H, k)
    out_h = hip.apply_hidden(to_dev(x), to_dev(w2), to_dev(h), seg, to_dev(g), H, k)
    torch.cuda.synchronize()
    xp = O.token_proj(x, w2, dt)
    slot = to_host(seg["pair_slot"])
    ref = O.apply(xp, O.to_f32(h, dt)[:U], O.to_f32(v, dt)[:U], slot, g, H, k, dt)
    check_out(O.to_f32(to_host(out), dt), ref, dt, signal=True, nerr_max=2e-3)
    ref_h = O.apply_hidden(xp, O.to_f32(h, dt)[:U], w2, slot, g, H, k, dt)
    check_out(O.to_f32(to_host(out_h), dt), ref_h, dt, signal=True, nerr_max=2e-3)


@pytest.mark.parametrize("d,dh,H,dt", [(1024, 128, 8, "bf16"), (4096, 64, 2, "bf16"), (256, 64, 3, "fp32")])
def test_scatter_paths_bit_identical(d, dh, H, dt):
    """The scatter-back's three forms give the same bits: up to 1,024 tokens one workgroup
    per token with the head rows in LDS (d 1024 bf16, d 256 fp32) or, for rows too wide
    for it, the head kernel plus the head sum (d 4096); above 1,024 tokens one wave per
    token.  The hidden and v rows are functions of the expert id, so the first 1,024
    tokens of a 1,025-token call must give the output of a call on those 1,024 tokens."""
    rng = np.random.default_rng(d + H)
    k, E = 4, 3000
    enc = (lambda a: O.f32_to_bf16_bits(a)) if dt == "bf16" else (lambda a: a.astype(np.float32))
    x = enc(rng.standard_normal((1025, d)).astype(np.float32))
    w2 = enc((rng.uniform(-1, 1, (2 * d, dh)) * 4 / np.sqrt(d)).astype(np.float32))
    ids = rng.integers(0, E, (1025, H, k)).astype(np.int32)
    g = enc(rng.uniform(0, 1, (1025, H, k)).astype(np.float32))
    h_e = enc(rng.standard_normal((E, dh)).astype(np.float32) * 0.3)
    v_e = enc(rng.standard_normal((E, d)).astype(np.float32))
    outs = []
    for n in (1025, 1024):
        seg = hip.sort_segment(to_dev(ids[:n].reshape(-1)), E)
        U = int(seg["n_unique"].item())
        uniq = to_host(seg["uniq"])[:U]
        h = np.zeros((seg["max_unique"], dh), h_e.dtype)
        v = np.zeros((seg["max_unique"], d), v_e.dtype)
        h[:U], v[:U] = h_e[uniq], v_e[uniq]
        out = hip.apply_scatter(to_dev(x[:n]), to_dev(w2), to_dev(h), to_dev(v), seg, to_dev(g[:n]), H, k)
        torch.cuda.synchronize()
        outs.append(to_host(out))
    assert np.array_equal(outs[0][:1024], outs[1])


def _stress_case(kind, rng, rows, K, dh2, dt):
    """Adversarial query / sub-key sets for the certified routing filter."""
    q = rng.standard_normal((rows, 2 * dh2)).astype(np.float32)
    k1 = rng.standard_normal((K, dh2)).astype(np.float32) / np.sqrt(dh2)
    k2 = rng.standard_normal((K, dh2)).astype(np.float32) / np.sqrt(dh2)
    if kind == "all_equal":        # every sub-key identical: all K scores tie
        k1[:] = k1[0]
        k2[:] = k2[3]
    elif kind == "near_ties":      # keys differ by tiny perturbations -> scores within a few ulps
        k1 = k1[:1] + 1e-3 * k1
        k2 = k2[:1] + 1e-3 * k2
    elif kind == "cancellation":   # large terms cancelling: |s| << ||q|| ||k||
        k1[:, dh2 // 2:] = -k1[:, : dh2 // 2] if dh2 % 2 == 0 else k1[:, dh2 // 2:]
        q[:, dh2 // 2: dh2] = q[:, : dh2 // 2] * (1 + 1e-3 * rng.standard_normal((rows, dh2 // 2)))
    elif kind == "zipf":           # sub-key rows scaled by (r+1)^-1.1
        z = (np.arange(K) + 1.0) ** -1.1
        k1 *= z[:, None]
        k2 *= z[:, None]
    elif kind == "mixed":          # one wave's rows: all scores tied / cancelling / plain
        h = dh2 // 2
        k1[:, h:2 * h] = -k1[:, :h]
        q[1::3] = 0.0
        q[2::3, h:2 * h] = q[2::3, :h] * (1 + 1e-3 * rng.standard_normal((len(q[2::3]), h)))
    elif kind == "dynamic_range":  # magnitudes spread over many binades
        q *= np.exp2(rng.integers(-20, 20, q.shape)).astype(np.float32)
        k1 *= np.exp2(rng.integers(-10, 10, k1.shape)).astype(np.float32)
    enc = (lambda a: O.f32_to_bf16_bits(a)) if dt == "bf16" else (lambda a: a.astype(np.float32))
    return enc(q), enc(k1), enc(k2)


@pytest.mark.parametrize("dt", ["bf16", "fp32"])
@pytest.mark.parametrize("kind", ["all_equal", "near_ties", "cancellation", "zipf", "dynamic_range", "mixed"])
def test_route_stress_bit_exact(kind, dt):
    rng = np.random.default_rng(hash((kind, dt)) % 2**32)
    rows, K, dh2, top_k = 96, 512, 128, 16
    q, k1, k2 = _stress_case(kind, rng, rows, K, dh2, dt)
    g_ref, ids_ref = O.route(q, k1, k2, top_k, dt)
    for norms in (None, "host"):
        kn = None
        if norms == "host":
            from ethos_amd import hip as H

            kn = H.key_norm_bounds(to_dev(k1), to_dev(k2)).cuda()
        g, ids = hip.route_topk(to_dev(q), to_dev(k1), to_dev(k2), top_k, key_norms=kn)
        torch.cuda.synchronize()
        got = to_host(ids)
        assert np.array_equal(got, ids_ref), f"{kind}/{dt}/{norms}: {np.sum(np.any(got != ids_ref, -1))} rows differ"
        # the gates too, bit for bit (same ids, same list order, same softmax contract)
        gg, gr = O.to_f32(to_host(g), dt), O.to_f32(g_ref, dt)
        assert np.array_equal(gg, gr), f"{kind}/{dt}/{norms}: {np.sum(np.any(gg != gr, -1))} rows' gates differ"


@pytest.mark.parametrize("dl,dh,d,U", [(128, 256, 1024, 1000), (128, 512, 512, 300), (128, 512, 1024, 129),
                                        (128, 512, 1024, 1), (128, 512, 768, 3001), (128, 256, 320, 1000)])
def test_generate_shapes(dl, dh, d, U):
    """Generator over shapes the configs do not hit (hidden 256, 512- and 768-wide models
    (two and three 256-column groups), a 320-wide model (not a multiple of 256 columns),
    tile remainders and a single expert)."""
    rng = np.random.default_rng(dl + dh + d + U)
    E = 5000
    lat = O.f32_to_bf16_bits(rng.standard_normal((E, dl)).astype(np.float32))
    w1 = O.f32_to_bf16_bits((rng.uniform(-1, 1, (dh, dl)) * 4 / np.sqrt(dl)).astype(np.float32))
    w2 = O.f32_to_bf16_bits((rng.uniform(-1, 1, (2 * d, dh)) * 4 / np.sqrt(dh)).astype(np.float32))
    uniq = np.sort(rng.choice(E, U, replace=False)).astype(np.int32)
    h_ref, v_ref = O.generate(lat, uniq, w1, w2, "bf16")
    h, v = _generate(lat, uniq, w1, w2, U + 3, "bf16")
    _check_rows(h[:U], h_ref, "bf16")
    _check_rows(v[:U], v_ref, "bf16")


@pytest.mark.parametrize("dh", [512, 256])
def test_generate_v_row_kernels_agree(dh):
    """The v-row kernel for widths that are multiples of 256 columns (W_v rows resident,
    each tile's epilogue during the next tile's products) and the one for other widths
    (hidden rows resident) use the same operands and k order per output column, so a
    320-wide model with W_v's first 320 rows gives the 1024-wide model's first 320 columns
    bit for bit."""
    rng = np.random.default_rng(dh)
    E, dl, d, U = 3000, 128, 1024, 2500
    lat = O.f32_to_bf16_bits(rng.standard_normal((E, dl)).astype(np.float32))
    w1 = O.f32_to_bf16_bits((rng.uniform(-1, 1, (dh, dl)) * 4 / np.sqrt(dl)).astype(np.float32))
    w2 = O.f32_to_bf16_bits((rng.uniform(-1, 1, (2 * d, dh)) * 4 / np.sqrt(dh)).astype(np.float32))
    uniq = np.sort(rng.choice(E, U, replace=False)).astype(np.int32)
    dn = 320
    w2n = np.concatenate([w2[:dn], w2[d:d + dn]])
    h, v = _generate(lat, uniq, w1, w2, U, "bf16")
    hn, vn = _generate(lat, uniq, w1, w2n, U, "bf16")
    assert np.array_equal(h[:U], hn[:U])
    assert np.array_equal(v[:U, :dn], vn[:U]), int(np.sum(v[:U, :dn] != vn[:U]))


@pytest.mark.parametrize("dl,dh,d,dt", [(16, 32, 64, "fp32"), (16, 32, 64, "bf16"), (128, 512, 1024, "bf16"),
                                         (128, 512, 320, "bf16")])
def test_generate_clamps_unique_count(dl, dh, d, dt):
    """A device unique-expert count above max_unique (the rows uniq, h and v hold) is
    clamped: rows below max_unique are generated, nothing past the buffers is touched.
    Covers the generic kernel (fp32, d_latent 16), the W-stationary kernels (d 1024) and
    the H-stationary expand (d 320)."""
    rng = np.random.default_rng(dl + dh + d)
    E, max_u = 2000, 100
    enc = (lambda a: O.f32_to_bf16_bits(a)) if dt == "bf16" else (lambda a: a.astype(np.float32))
    lat = enc(rng.standard_normal((E, dl)).astype(np.float32))
    w1 = enc((rng.uniform(-1, 1, (dh, dl)) * 4 / np.sqrt(dl)).astype(np.float32))
    w2 = enc((rng.uniform(-1, 1, (2 * d, dh)) * 4 / np.sqrt(dh)).astype(np.float32))
    uniq = np.sort(rng.choice(E, max_u, replace=False)).astype(np.int32)
    n_unique = torch.tensor([3 * max_u], dtype=torch.int32, device="cuda")
    h, v = hip.generate(to_dev(lat), to_dev(uniq), n_unique, max_u, to_dev(w1), to_dev(w2))
    torch.cuda.synchronize()
    h_ref, v_ref = O.generate(lat, uniq, w1, w2, dt)
    _check_rows(O.to_f32(to_host(h), dt), h_ref, dt)
    _check_rows(O.to_f32(to_host(v), dt), v_ref, dt)


@pytest.mark.parametrize("dh", [512, 256])
def test_generate_many_tiles(dh):
    """Enough experts that each workgroup runs several whole tiles back to back plus the
    column-split last round (whose first part alone stores the hidden rows); sampled
    rows against the oracle."""
    rng = np.random.default_rng(dh)
    E, dl, d, U = 262144, 128, 1024, 200070
    lat = O.f32_to_bf16_bits(rng.standard_normal((E, dl)).astype(np.float32))
    w1 = O.f32_to_bf16_bits((rng.uniform(-1, 1, (dh, dl)) * 4 / np.sqrt(dl)).astype(np.float32))
    w2 = O.f32_to_bf16_bits((rng.uniform(-1, 1, (2 * d, dh)) * 4 / np.sqrt(dh)).astype(np.float32))
    uniq = np.sort(rng.choice(E, U, replace=False)).astype(np.int32)
    h, v = _generate(lat, uniq, w1, w2, U + 5, "bf16")
    edges = [0, 1, 255, 256, 257, 65535, 65536, 131071, 131072, 196607, 196608, U - 2, U - 1]
    rows = np.unique(np.concatenate([edges, rng.choice(U, 587, replace=False)])).astype(np.int64)
    h_ref, v_ref = O.generate(lat, uniq[rows], w1, w2, "bf16")
    _check_rows(h[rows], h_ref, "bf16")
    _check_rows(v[rows], v_ref, "bf16")


@pytest.mark.parametrize("n", [96, 200])
@pytest.mark.parametrize("kind", ["cancellation", "midpoints", "binades", "subnormals", "zero_rows", "ragged_d"])
def test_query_proj_certified_fallback_bit_exact(kind, n):
    """Inputs aimed at the certificate: cancellation and rounding ties (most elements go
    to the exact fp64 recomputation), elements spread over many binades (not exact in the
    per-row digit format), subnormals, all-zero rows against negative-zero bias and
    BatchNorm shift, and a model width that is not a multiple of the 64-byte K chunk.  The
    result must equal the oracle bit for bit, for 96 tokens (the reduction split over
    workgroups, partial sums added by a second kernel) and 200 (one workgroup per tile)."""
    rng = np.random.default_rng(11)
    d, H, dq = 512, 2, 64
    if kind == "ragged_d":
        d = 200
    if kind in ("binades", "subnormals", "zero_rows", "ragged_d"):
        x = rng.standard_normal((n, d)).astype(np.float32)
        w = rng.uniform(-1, 1, (H, dq, d)).astype(np.float32) / np.sqrt(d)
        b = rng.uniform(-0.1, 0.1, (H, dq)).astype(np.float32)
        if kind == "binades":
            x *= np.exp2(rng.integers(-24, 8, x.shape)).astype(np.float32)
            w *= np.exp2(rng.integers(-24, 8, w.shape)).astype(np.float32)
        elif kind == "subnormals":
            tiny = rng.random(x.shape) < 0.2
            x[tiny] = (rng.integers(-127, 128, int(tiny.sum())) * 2.0 ** -133).astype(np.float32)
            x[::7] *= 2.0 ** -120
            w[0, :4] = (rng.integers(-127, 128, (4, d)) * 2.0 ** -133).astype(np.float32)
        elif kind == "zero_rows":
            x[::3] = 0.0
            b[:, ::2] = -0.0
    elif kind == "cancellation":
        half = rng.standard_normal((n, d // 2)).astype(np.float32)
        x = np.concatenate([half, half], axis=1)
        a = rng.uniform(-1, 1, (H, dq, d // 2)).astype(np.float32) / np.sqrt(d)
        w = np.concatenate([a, -a + 1e-3 * rng.standard_normal(a.shape).astype(np.float32)], axis=2)
        b = np.zeros((H, dq), np.float32)
    else:
        # small integers make many exact products and sums land on bf16 rounding ties
        x = rng.integers(-8, 9, (n, d)).astype(np.float32)
        w = rng.integers(-8, 9, (H, dq, d)).astype(np.float32) / 64
        b = rng.integers(-4, 5, (H, dq)).astype(np.float32) / 128
    x, w, b = (O.f32_to_bf16_bits(v) for v in (x, w, b))
    alpha = rng.uniform(0.5, 1.5, (H, dq)).astype(np.float32)
    beta = rng.uniform(-0.1, 0.1, (H, dq)).astype(np.float32)
    if kind == "zero_rows":
        beta[:, ::4] = -0.0
        beta[:, 1::4] = 0.0
    q_ref = O.query_proj(x, w, b, alpha, beta, "bf16")
    wd = to_dev(w)
    q = hip.query_proj(to_dev(x), wd, to_dev(b), to_dev(alpha), to_dev(beta))
    qp = hip.query_proj(to_dev(x), wd, to_dev(b), to_dev(alpha), to_dev(beta), prepared=hip.query_proj_prepare(wd))
    torch.cuda.synchronize()
    assert np.array_equal(to_host(q), q_ref), f"{np.sum(to_host(q) != q_ref)} elements differ"
    assert np.array_equal(to_host(qp), q_ref), f"prepared weights: {np.sum(to_host(qp) != q_ref)} elements differ"


@pytest.mark.parametrize("name,signal", [("tiny", False), ("tiny", True), ("tiny_fp32", True), ("cfg1", False),
                                         ("cfg3", True), ("cfg3", False)])
def test_apply_hidden_matches_oracle(name, signal):
    """Hidden-space reordering through the C-ABI: hidden-only generation gives the same h
    rows as the full generator, and the apply matches the oracle's Algorithm-1 form (fp32: to
    1e-4; bf16: the stated tolerance, mostly identical elements) and the scatter form within
    the bf16 tolerance of the layer."""
    sh, x, P = _setup(name, signal=signal)
    q = O.query_proj(x, P["Wq"], P["bq"], P["alpha"], P["beta"], sh.dtype)
    g, ids = O.route(q, P["K1"], P["K2"], sh.top_k, sh.dtype)
    seg = hip.sort_segment(to_dev(ids.reshape(-1)), sh.num_experts)
    U = int(seg["n_unique"].item())
    w2 = to_dev(P["W2"])
    args = (to_dev(P["latents"]), seg["uniq"], seg["n_unique"], seg["max_unique"], to_dev(P["W1"]), w2)
    h_only, none = hip.generate(*args, with_v=False)
    h_dev, v_dev = hip.generate(*args)
    out = hip.apply_hidden(to_dev(x), w2, h_only, seg, to_dev(g), sh.num_heads, sh.top_k)
    torch.cuda.synchronize()
    assert none is None and torch.equal(h_only[:U], h_dev[:U])
    h = O.to_f32(to_host(h_dev), sh.dtype)[:U]
    v = O.to_f32(to_host(v_dev), sh.dtype)[:U]
    xp = O.token_proj(x, P["W2"], sh.dtype)
    slot = to_host(seg["pair_slot"])
    ref = O.apply_hidden(xp, h, P["W2"], slot, g, sh.num_heads, sh.top_k, sh.dtype)
    got = O.to_f32(to_host(out), sh.dtype)
    check_out(got, ref, sh.dtype, signal=signal, nerr_max=2e-3)
    if sh.dtype == "bf16":
        assert np.mean(got == ref) > 0.9
    scatter = O.apply(xp, h, v, slot, g, sh.num_heads, sh.top_k, sh.dtype)
    check_out(got, scatter, sh.dtype, signal=signal, nerr_max=1e-2)


@pytest.mark.parametrize("n_tok,d,dh,dt", [(100, 1024, 512, "bf16"), (37, 256, 128, "bf16"), (70, 96, 64, "bf16"),
                                           (33, 128, 96, "fp32"), (5, 4096, 256, "bf16")])
def test_apply_hidden_shapes(n_tok, d, dh, dt):
    """Hidden-space apply over shapes the configs do not hit: the MFMA projection (d_hidden a
    multiple of 64), the generic transposed projection (d_hidden = 96) and d_model 4096."""
    rng = np.random.default_rng(n_tok + d + dh + 1)
    H, k, E = 2, 4, 300
    enc = (lambda a: O.f32_to_bf16_bits(a)) if dt == "bf16" else (lambda a: a.astype(np.float32))
    x = enc(rng.standard_normal((n_tok, d)).astype(np.float32))
    w2 = enc((rng.uniform(-1, 1, (2 * d, dh)) * 4 / np.sqrt(d)).astype(np.float32))
    ids = rng.integers(0, E, (n_tok, H, k)).astype(np.int32)
    g = enc(rng.uniform(0, 1, (n_tok, H, k)).astype(np.float32))
    seg = hip.sort_segment(to_dev(ids.reshape(-1)), E)
    U = int(seg["n_unique"].item())
    h = enc(rng.standard_normal((seg["max_unique"], dh)).astype(np.float32) * 0.3)
    out = hip.apply_hidden(to_dev(x), to_dev(w2), to_dev(h), seg, to_dev(g), H, k)
    torch.cuda.synchronize()
    xp = O.token_proj(x, w2, dt)
    ref = O.apply_hidden(xp, O.to_f32(h, dt)[:U], w2, to_host(seg["pair_slot"]), g, H, k, dt)
    got = O.to_f32(to_host(out), dt)
    check_out(got, ref, dt, signal=True, nerr_max=2e-3)


@pytest.mark.parametrize("name", ["tiny", "tiny_fp32", "cfg1", "cfg3", "cfg2"])
@pytest.mark.parametrize("hidden_space", [False, True])
def test_expert_forward_matches_separate_calls(name, hidden_space):
    """ethos_expert_forward (one call, activations between the generator's kernels, W_u^T
    from the caller for bf16) against ethos_generate followed by ethos_apply_scatter /
    ethos_apply_hidden: bit-identical outputs and hidden rows."""
    sh, x, P = _setup(name, signal=True)
    q = O.query_proj(x, P["Wq"], P["bq"], P["alpha"], P["beta"], sh.dtype)
    gates, ids = O.route(q, P["K1"], P["K2"], sh.top_k, sh.dtype)
    seg = hip.sort_segment(to_dev(ids.reshape(-1)), sh.num_experts)
    xd, lat, w1, w2, g = (to_dev(a) for a in (x, P["latents"], P["W1"], P["W2"], gates))
    h, v = hip.generate(lat, seg["uniq"], seg["n_unique"], seg["max_unique"], w1, w2, with_v=not hidden_space)
    if hidden_space:
        want = hip.apply_hidden(xd, w2, h, seg, g, sh.num_heads, sh.top_k)
    else:
        want = hip.apply_scatter(xd, w2, h, v, seg, g, sh.num_heads, sh.top_k)
    wut = w2[: sh.d_model].t().contiguous() if sh.dtype == "bf16" else None
    got, h2 = hip.expert_forward(xd, lat, w1, w2, seg, g, sh.num_heads, sh.top_k, hidden_space=hidden_space, wut=wut)
    got_nowut, _ = hip.expert_forward(xd, lat, w1, w2, seg, g, sh.num_heads, sh.top_k, hidden_space=hidden_space)
    # the token projection computed beforehand (ethos_token_proj) and passed in
    xp = hip.token_proj(xd, w2, wut)
    got_xp, _ = hip.expert_forward(xd, lat, w1, w2, seg, g, sh.num_heads, sh.top_k, hidden_space=hidden_space,
                                   wut=wut, xp=xp)
    torch.cuda.synchronize()
    U = int(seg["n_unique"].item())
    assert np.array_equal(to_host(h2)[:U], to_host(h)[:U])
    assert np.array_equal(to_host(got), to_host(want))
    assert np.array_equal(to_host(got_nowut), to_host(want))
    assert np.array_equal(to_host(got_xp), to_host(want))
    # x_proj itself: fp32 MFMA accumulation rounded once, against the oracle's fp64 product
    # rounded once -- one rounding step apart, plus the fp32 accumulation error on
    # cancelling sums
    xr = O.to_f32(O.token_proj(x, P["W2"], sh.dtype), sh.dtype)
    xg = O.to_f32(to_host(xp), sh.dtype)
    ulp = 2.0 ** -7 if sh.dtype == "bf16" else 2.0 ** -22
    bad = np.abs(xg - xr) > ulp * np.abs(xr) + 2.0 ** -16 * np.abs(xr).max()
    assert not bad.any(), (f"{bad.sum()} of {bad.size}; shapes {xg.shape} {xr.shape}; first {np.argwhere(bad)[:3]} "
                           f"got {xg[bad][:3]} want {xr[bad][:3]}")


@pytest.mark.parametrize("hidden_space", [False, True])
def test_expert_forward_hot_experts(hidden_space):
    """Routing with four hot experts among ~10^5 others (1,024 tokens, 131,072 pairs): the
    hidden-row kernel computes the activations of tiles of at most 2,048 pairs (64 unique
    experts per tile) and the activation kernel the pairs of larger tiles.  Here two tiles
    are over that cap (3,277 and 2,149 pairs of one expert) and one just under it.  The one
    call must equal generate + apply bit for bit, and the apply must meet the oracle on a
    token sample (given the same hidden and v rows)."""
    sh = SHAPES["cfg2"].with_tokens(1024)
    xt, sd = make_inputs(sh, signal=True)
    P = O.unpack_state(sd, sh.num_heads)
    x = O.from_torch(xt)
    n, H, k, E = sh.n_tok, sh.num_heads, sh.top_k, sh.num_experts
    rng = np.random.default_rng(5)
    ids = rng.integers(0, E, size=n * H * k).astype(np.int32)
    p = np.arange(ids.size)
    for mod, rem, e in ((40, 0, 7777), (61, 3, 150000), (70, 1, 100000), (300, 2, 200000)):
        ids[p % mod == rem] = e
    gates = O.f32_to_bf16_bits((rng.random(ids.size) / 16).astype(np.float32)).reshape(n, H, k)
    seg = hip.sort_segment(to_dev(ids), E)
    U = int(seg["n_unique"].item())
    off = to_host(seg["seg_off"])[: U + 1].astype(np.int64)
    tile_pairs = off[np.minimum(np.arange(0, U, 64) + 64, U)] - off[np.arange(0, U, 64)]
    assert U * sh.d_hidden * 2 > 8 << 20, "the activations must take the expert order"
    assert (tile_pairs > 2048).sum() == 2 and ((tile_pairs > 1800) & (tile_pairs <= 2048)).sum() >= 1, tile_pairs.max()
    xd, lat, w1, w2, g = (to_dev(a) for a in (x, P["latents"], P["W1"], P["W2"], gates))
    h, v = hip.generate(lat, seg["uniq"], seg["n_unique"], seg["max_unique"], w1, w2, with_v=not hidden_space)
    if hidden_space:
        want = hip.apply_hidden(xd, w2, h, seg, g, H, k)
    else:
        want = hip.apply_scatter(xd, w2, h, v, seg, g, H, k)
    wut = w2[: sh.d_model].t().contiguous()
    got, h2 = hip.expert_forward(xd, lat, w1, w2, seg, g, H, k, hidden_space=hidden_space, wut=wut)
    torch.cuda.synchronize()
    assert np.array_equal(to_host(h2)[:U], to_host(h)[:U])
    assert np.array_equal(to_host(got), to_host(want))
    # the apply against the oracle on tokens that use the hot experts (and others)
    tokens = np.array([0, 1, 5, 17, 300, 511, 777, 1023])
    xp = O.token_proj(x, P["W2"], sh.dtype)
    hh = O.to_f32(to_host(h), sh.dtype)[:U]
    slot = to_host(seg["pair_slot"])
    if hidden_space:
        ref = O.apply_hidden(xp, hh, P["W2"], slot, gates, H, k, sh.dtype, tokens=tokens)
    else:
        ref = O.apply(xp, hh, O.to_f32(to_host(v), sh.dtype)[:U], slot, gates, H, k, sh.dtype, tokens=tokens)
    check_out(O.to_f32(to_host(got), sh.dtype)[tokens], ref, sh.dtype, signal=True, nerr_max=2e-3)


def test_stage_events_recorded_in_expert_forward():
    """Five events per ethos_expert_forward call, recorded in order on the launch stream."""
    sh, x, P = _setup("cfg3", signal=True)
    q = O.query_proj(x, P["Wq"], P["bq"], P["alpha"], P["beta"], sh.dtype)
    gates, ids = O.route(q, P["K1"], P["K2"], sh.top_k, sh.dtype)
    seg = hip.sort_segment(to_dev(ids.reshape(-1)), sh.num_experts)
    args = [to_dev(a) for a in (x, P["latents"], P["W1"], P["W2"])]
    g = to_dev(gates)
    start = torch.cuda.Event(enable_timing=True)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
    for e in evs:
        e.record()
    torch.cuda.synchronize()
    start.record()
    hip.stage_events(evs)
    hip.expert_forward(*args, seg, g, sh.num_heads, sh.top_k)
    hip.stage_events([])
    end = torch.cuda.Event(enable_timing=True)
    end.record()
    torch.cuda.synchronize()
    marks = [start] + evs + [end]
    gaps = [a.elapsed_time(b) for a, b in zip(marks, marks[1:])]
    assert all(t >= 0 for t in gaps), gaps
    assert sum(gaps[:-1]) > 0


@pytest.mark.parametrize("n_tok,H,k,d,dh,E,dt", [(64, 8, 16, 1024, 512, 262144, "bf16"),   # one launch
                                                 (5, 2, 3, 256, 128, 300, "bf16"),         # one launch, one tile
                                                 (64, 2, 4, 96, 64, 300, "bf16"),          # d % 64: two launches
                                                 (1100, 8, 16, 256, 128, 262144, "bf16"),  # tiled sort: two launches
                                                 (33, 2, 4, 128, 96, 300, "fp32")])
def test_sort_segment_token_proj_matches_separate_calls(n_tok, H, k, d, dh, E, dt):
    """The sort with the token projection beside it gives the outputs of sort_segment and
    token_proj bit for bit, whether it runs as one launch (small bf16 batches) or as the two
    in turn."""
    rng = np.random.default_rng(n_tok + d)
    enc = (lambda a: O.f32_to_bf16_bits(a)) if dt == "bf16" else (lambda a: a.astype(np.float32))
    x = to_dev(enc(rng.standard_normal((n_tok, d)).astype(np.float32)))
    w2 = to_dev(enc((rng.uniform(-1, 1, (2 * d, dh)) / np.sqrt(d)).astype(np.float32)))
    wut = w2[:d].t().contiguous() if dt == "bf16" else None
    ids = to_dev(rng.integers(0, E, n_tok * H * k).astype(np.int32))
    seg, xp = hip.sort_segment_token_proj(ids, E, x, w2, wut)
    seg_ref = hip.sort_segment(ids, E)
    xp_ref = hip.token_proj(x, w2, wut)
    torch.cuda.synchronize()
    U = int(seg_ref["n_unique"].item())
    assert int(seg["n_unique"].item()) == U
    for key in ("perm", "pair_slot", "sorted_slot"):
        assert torch.equal(seg[key], seg_ref[key]), key
    assert torch.equal(seg["uniq"][:U], seg_ref["uniq"][:U]) and torch.equal(seg["seg_off"][:U + 1], seg_ref["seg_off"][:U + 1])
    assert torch.equal(xp, xp_ref)
