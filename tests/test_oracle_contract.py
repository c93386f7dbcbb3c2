"""Pins the CPU oracle against mathematics that does not depend on the oracle's own code.

Each check is chosen so a plausible slip fails it: a wrong rounding direction or
double rounding (exact rational rounding), an inexact accumulation (exact
rational dot products), a transposed decode or a wrong tie rule (exhaustive top-k
over all K^2 pairs), an unstable sort (numpy's stable argsort).
"""
from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as O


def _round_frac(x: Fraction, p: int) -> Fraction:
    """Round an exact rational to p significant bits, nearest with ties to even
    (normal range only)."""
    if x == 0:
        return Fraction(0)
    a = -x if x < 0 else x
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp = Fraction(2) ** (e - (p - 1))
    m = a / ulp
    fl = m.numerator // m.denominator
    rem = m - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    r = fl * ulp
    return -r if x < 0 else r


def _bf16_exact_round(x: Fraction) -> int:
    """bf16 bit pattern of the correctly rounded value of x."""
    f = np.float32(float(_round_frac(x, 8)))  # exactly representable
    return int(np.array([f]).view(np.uint32)[0] >> 16)


def test_f64_to_bf16_is_correctly_rounded():
    rng = np.random.default_rng(1)
    vals = list(rng.standard_normal(3000) * np.exp2(rng.integers(-20, 20, 3000)))
    # near-halfway cases: bf16 midpoints and their fp64 neighbours (double rounding traps)
    for _ in range(2000):
        b = int(rng.integers(0x0080, 0x7F00))
        lo = np.array([b << 16], np.uint32).view(np.float32)[0]
        hi = np.array([(b + 1) << 16], np.uint32).view(np.float32)[0]
        mid = (float(lo) + float(hi)) / 2
        vals += [mid, np.nextafter(mid, 0.0), np.nextafter(mid, np.inf), -mid]
        # fp32 midpoint that is not a bf16 midpoint, and values that round to odd
        vals.append(mid + (float(hi) - float(lo)) * 2.0 ** -20)
    for v in vals:
        want = _bf16_exact_round(Fraction(v))
        got = int(O.lib().ethos_oracle_f64_to_bf16(float(v)))
        assert got == want, (v, hex(got), hex(want))
    # the numpy twin used by the layer oracle agrees bit for bit
    arr = np.array(vals, np.float64)
    np_bits = O.f64_to_bf16_bits(arr)
    c_bits = np.array([O.lib().ethos_oracle_f64_to_bf16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(np_bits, c_bits)


def _exact_dot(a_f32, b_f32):
    return sum(Fraction(float(x)) * Fraction(float(y)) for x, y in zip(a_f32, b_f32))


@pytest.mark.parametrize("n", [64, 128, 256, 1024])
def test_dot64_exact_for_bf16(n):
    """For bf16 operands the fp64 FMA chain equals the exact rational dot product."""
    rng = np.random.default_rng(n)
    for _ in range(20):
        a = O.f32_to_bf16_bits(rng.standard_normal(n).astype(np.float32))
        b = O.f32_to_bf16_bits((rng.standard_normal(n) / 11).astype(np.float32))
        got = O.lib().ethos_oracle_dot64(O._p(a), O._p(b), n, 1)
        assert Fraction(got) == _exact_dot(O.to_f32(a, "bf16"), O.to_f32(b, "bf16"))


def test_query_proj_bf16_matches_exact_rational():
    rng = np.random.default_rng(7)
    n, d, H, dq = 5, 96, 2, 8
    x = O.f32_to_bf16_bits(rng.standard_normal((n, d)).astype(np.float32))
    Wq = O.f32_to_bf16_bits((rng.uniform(-1, 1, (H, dq, d)) / np.sqrt(d)).astype(np.float32))
    bq = O.f32_to_bf16_bits((rng.uniform(-1, 1, (H, dq)) / np.sqrt(d)).astype(np.float32))
    alpha = rng.uniform(0.5, 1.5, (H, dq)).astype(np.float32)
    beta = rng.uniform(-0.1, 0.1, (H, dq)).astype(np.float32)
    q = O.query_proj(x, Wq, bq, alpha, beta, "bf16")
    xf, wf, bf = O.to_f32(x, "bf16"), O.to_f32(Wq, "bf16"), O.to_f32(bq, "bf16")
    for t in range(n):
        for h in range(H):
            for o in range(dq):
                lin = _exact_dot(xf[t], wf[h, o]) + Fraction(float(bf[h, o]))
                ql = np.array([_bf16_exact_round(lin)], np.uint16)
                qlf = O.to_f32(ql, "bf16")[0]
                # BN: one fp32 fused multiply-add, then rounding to bf16
                fused = Fraction(float(qlf)) * Fraction(float(alpha[h, o])) + Fraction(float(beta[h, o]))
                f32 = np.float32(float(_round_frac(fused, 24)))
                want = O.f32_to_bf16_bits(np.array([f32]))[0]
                assert q[t, h, o] == want


def _brute_topk(s1, s2, K, top_k, dt):
    """Exhaustive canonical top-k over all K^2 pairs: (score desc, expert id asc)."""
    c = O.round_T((s1[:, None] + s2[None, :]).astype(np.float32), dt).reshape(-1)
    e = np.arange(K * K)
    order = np.lexsort((e, -c.astype(np.float64)))
    return e[order[:top_k]], c[order[:top_k]]


@pytest.mark.parametrize("K,top_k", [(16, 1), (16, 4), (64, 8), (32, 16)])
def test_select_equals_exhaustive_topk_without_ties(K, top_k):
    """With k_cand = 2k >= k and no ties, the candidate grid holds the global top-k
    over all K^2 products (a non-candidate row is dominated by k_cand >= k rows)."""
    rng = np.random.default_rng(K * 100 + top_k)
    rows = 64
    s1 = rng.standard_normal((rows, K)).astype(np.float32)
    s2 = rng.standard_normal((rows, K)).astype(np.float32)
    gates, ids = O.select(s1, s2, top_k, "fp32")
    for r in range(rows):
        want_e, want_c = _brute_topk(s1[r], s2[r], K, top_k, "fp32")
        assert np.array_equal(ids[r], want_e)
        # the softmax closed form, and the contract's exact fp32 form: the fp64 exponential
        # rounded once, an fp32 sum in list order, an fp32 divide
        d = (want_c - want_c[0]).astype(np.float64)
        np.testing.assert_allclose(gates[r], np.exp(d) / np.exp(d).sum(), rtol=2e-6)
        ex = np.exp(d).astype(np.float32)
        tot = np.float32(0)
        for e in ex:
            tot = np.float32(tot + e)
        assert np.array_equal(gates[r], (ex / tot).astype(np.float32))


def test_select_decode_uses_first_half_as_high_digit():
    """Expert id = (index in sub_keys_1) * K + (index in sub_keys_2)."""
    K = 8
    s1 = np.full((1, K), -10, np.float32)
    s2 = np.full((1, K), -10, np.float32)
    s1[0, 5] = 3.0
    s2[0, 2] = 2.0
    _, ids = O.select(s1, s2, 1, "fp32", k_cand=2)
    assert ids[0, 0] == 5 * K + 2


def test_select_tie_rule_lowest_index():
    K = 16
    s1 = np.zeros((1, K), np.float32)  # every sub-key ties
    s2 = np.zeros((1, K), np.float32)
    _, ids, cand = O.select(s1, s2, 4, "fp32", want_cand=True)
    assert list(cand[0, 0]) == list(range(8)) and list(cand[0, 1]) == list(range(8))
    assert list(ids[0]) == [0, 1, 2, 3]
    # ties that appear only after rounding the sum to bf16 break on expert id
    s1 = O.round_T(np.array([[1.0, 1.0 + 2**-7, 0.5, 0.25]], np.float32), "bf16")
    s2 = O.round_T(np.array([[2**-9, 0.0, -1.0, -2.0]], np.float32), "bf16")
    _, ids = O.select(s1, s2, 2, "bf16", k_cand=2)
    c = O.round_T((s1[0][:, None] + s2[0][None, :]).astype(np.float32), "bf16")
    e = np.arange(16)
    order = np.lexsort((e, -c.reshape(-1).astype(np.float64)))[:2]
    assert list(ids[0]) == list(order)


def test_single_expert_gate_is_one():
    rng = np.random.default_rng(3)
    s1 = rng.standard_normal((10, 32)).astype(np.float32)
    s2 = rng.standard_normal((10, 32)).astype(np.float32)
    for dt in ("fp32", "bf16"):
        g, _ = O.select(O.round_T(s1, dt), O.round_T(s2, dt), 1, dt)
        assert np.all(O.to_f32(g, dt) == 1.0)


def test_negative_zero_ties_positive_zero():
    s1 = np.array([[-0.0, 0.0, -1.0, -1.0]], np.float32)
    s2 = np.array([[0.0, -5.0, -5.0, -5.0]], np.float32)
    _, ids = O.select(s1, s2, 2, "fp32", k_cand=2)
    assert list(ids[0]) == [0 * 4 + 0, 1 * 4 + 0]


def test_route_rejects_bad_sizes():
    q = np.zeros((1, 8), np.float32)
    keys = np.zeros((4, 4), np.float32)
    with pytest.raises(ValueError):
        O.route(q, keys, keys, top_k=4, dt="fp32")  # k_cand 8 > K 4


@pytest.mark.parametrize("n,E", [(1, 1), (1000, 7), (5000, 4096), (20000, 262144), (3, 262144)])
def test_sort_segment_is_stable_counting_sort(n, E):
    rng = np.random.default_rng(n)
    ids = rng.integers(0, E, n).astype(np.int32)
    if n == 1000:
        ids[:500] = 3  # one long segment
    perm, uniq, seg, inv = O.sort_segment(ids, E)
    assert np.array_equal(perm, np.argsort(ids, kind="stable"))
    u, counts = np.unique(ids, return_counts=True)
    assert np.array_equal(uniq, u)
    assert np.array_equal(np.diff(seg), counts) and seg[0] == 0 and seg[-1] == n
    assert np.array_equal(uniq[inv], ids)


def test_sort_segment_rejects_out_of_range():
    with pytest.raises(ValueError):
        O.sort_segment(np.array([0, 5], np.int32), 5)


@pytest.mark.parametrize("H,k,d,dh", [(2, 4, 64, 32), (4, 8, 96, 64)])
def test_apply_hidden_is_apply_by_linearity(H, k, d, dh):
    """sum_p a_p (h_s W_v^T) = (sum_p a_p h_s) W_v^T: in fp32 with h_acc kept in float32 the
    hidden-space form equals the scatter form to float32 rounding; a missing head average,
    the W_u half in place of W_v or a transposed W_v does not."""
    rng = np.random.default_rng(H * k + d)
    n, U = 24, 40
    xp = rng.standard_normal((n, dh)).astype(np.float32)
    h = rng.standard_normal((U, dh)).astype(np.float32)
    W2 = (rng.standard_normal((2 * d, dh)) / np.sqrt(dh)).astype(np.float32)
    v = (h.astype(np.float64) @ W2[d:].astype(np.float64).T).astype(np.float32)
    slot = rng.integers(0, U, n * H * k).astype(np.int32)
    gates = rng.uniform(0, 1, (n, H, k)).astype(np.float32)
    ref = O.apply(xp, h, v, slot, gates, H, k, "fp32").astype(np.float64)
    got = O.apply_hidden(xp, h, W2, slot, gates, H, k, "fp32", hacc_round="none").astype(np.float64)
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() <= 1e-5 * scale
    wrong = O.apply_hidden(xp, h, np.concatenate([W2[d:], W2[:d]]), slot, gates, H, k, "fp32", hacc_round="none")
    assert np.abs(wrong - ref).max() > 1e-2 * scale
