"""CPU oracle for the ETHOS expert-layer forward path -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg import
this module, and only as the checker.  The product (``ethos_amd``) never imports
it and has no CPU fallback.

Layout of the oracle:
  * ethos_oracle.c (via ctypes): the exactly specified integer / rounding parts --
    query projection + eval BatchNorm, sub-key scoring, canonical top-k selection,
    softmax gates, and the stable reordering of pairs by expert id.
  * this file (numpy, fp64): the dense floating-point parts -- the expert
    generation network and the expert apply / weighted scatter-back -- with the
    layer dtype's rounding points placed where the reference rounds
    (model.py:320-341).

Reference algorithm (wrmedford/ETHOS):
  router            model.py:208-254
  generation net    model.py:168-179 (weights read directly at model.py:297-300)
  expert loop       model.py:306-341 (per pair: h = gelu(z W1); x_proj = x W_u;
                    a = gelu(h . x_proj) g; y += a * (h W_v); per-head fp32
                    accumulate, cast, head sum in dtype, divide by H)
The functions below keep the reference's intermediates: the hidden row h_e of each
unique expert, the token projection x_proj = x W_u (W_u = W2[:d_model]^T, the same for
every pair of a token) and v_e = h_e W_v (W_v = W2[d_model:]^T), each rounded to the
layer dtype where the reference rounds it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np
from scipy.special import erfc

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(HERE, "libethos_oracle.so")
DT_CODE = {"fp32": 0, "bf16": 1}

_lib = None


def build(force: bool = False) -> str:
    """Compile the C part of the oracle with gcc (oracle/Makefile)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(_LIB_PATH)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.ethos_oracle_query_proj.argtypes = [vp, vp, vp, vp, vp, i64, i32, i32, i32, i32, vp]
        L.ethos_oracle_query_proj.restype = None
        L.ethos_oracle_subkey_scores.argtypes = [vp, vp, i64, i32, i32, i32, i32, vp]
        L.ethos_oracle_subkey_scores.restype = None
        L.ethos_oracle_route.argtypes = [vp, vp, vp, i64, i32, i32, i32, i32, i32, vp, vp, vp]
        L.ethos_oracle_route.restype = ctypes.c_int
        L.ethos_oracle_select.argtypes = [vp, vp, i64, i32, i32, i32, i32, vp, vp, vp]
        L.ethos_oracle_select.restype = ctypes.c_int
        L.ethos_oracle_sort_segment.argtypes = [vp, i64, i64, vp, vp, vp, vp]
        L.ethos_oracle_sort_segment.restype = ctypes.c_int64
        L.ethos_oracle_f64_to_bf16.argtypes = [ctypes.c_double]
        L.ethos_oracle_f64_to_bf16.restype = ctypes.c_uint16
        L.ethos_oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        L.ethos_oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.ethos_oracle_dot64.argtypes = [vp, vp, i32, i32]
        L.ethos_oracle_dot64.restype = ctypes.c_double
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.c_void_p)


# ------------------------------------------------------------------ dtype helpers
# A dtype-T array is held as np.uint16 bit patterns for bf16 and np.float32 for fp32.

def bf16_bits_to_f32(u16: np.ndarray) -> np.ndarray:
    return (u16.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(f: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns."""
    b = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = (b + np.uint32(0x7FFF) + ((b >> 16) & 1)) >> 16
    r = np.where(nan, (b >> 16) | 0x40, r)
    return r.astype(np.uint16)


def f64_to_bf16_bits(d: np.ndarray) -> np.ndarray:
    """Correctly rounded float64 -> bf16 (round to odd at fp32, then nearest even)."""
    d = np.asarray(d, dtype=np.float64)
    f = d.astype(np.float32)
    b = f.view(np.uint32).copy()
    inexact = (f.astype(np.float64) != d) & np.isfinite(f)
    even = (b & 1) == 0
    adj = inexact & even
    toward_zero = np.abs(f.astype(np.float64)) > np.abs(d)
    b = np.where(adj & toward_zero, b - np.uint32(1), np.where(adj, b + np.uint32(1), b)).astype(np.uint32)
    return f32_to_bf16_bits(b.view(np.float32))


def to_f32(a: np.ndarray, dt: str) -> np.ndarray:
    return bf16_bits_to_f32(a) if dt == "bf16" else np.asarray(a, dtype=np.float32)


def round_T(v: np.ndarray, dt: str) -> np.ndarray:
    """Round fp64/fp32 values to dtype T; returns float32 holding the T values."""
    if dt == "bf16":
        if v.dtype == np.float32:
            return bf16_bits_to_f32(f32_to_bf16_bits(v))
        return bf16_bits_to_f32(f64_to_bf16_bits(v))
    return np.asarray(v).astype(np.float32)


def from_torch(t) -> np.ndarray:
    """CPU torch tensor -> numpy array in the storage convention above."""
    import torch

    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    if t.dtype == torch.float32:
        return t.numpy().copy()
    if t.dtype in (torch.int32, torch.int64):
        return t.numpy().copy()
    raise TypeError(f"unsupported dtype {t.dtype}")


def storage(a_f32: np.ndarray, dt: str) -> np.ndarray:
    """float32 array of T values -> storage convention."""
    return f32_to_bf16_bits(a_f32) if dt == "bf16" else np.ascontiguousarray(a_f32, dtype=np.float32)


def gelu64(v: np.ndarray) -> np.ndarray:
    """Exact (erf) GELU in fp64 -- F.gelu's default, model.py:174,323,329:
    0.5 v (1 + erf(v / sqrt 2)), evaluated as 0.5 v erfc(-v / sqrt 2), the same function
    without the cancellation of 1 + erf(.) for negative v."""
    return 0.5 * v * erfc(-v / np.sqrt(2.0))


# ------------------------------------------------------------------ router
def bn_coeffs(weight, bias, running_mean, running_var, eps: float = 1e-5):
    """fp32 eval-mode BatchNorm coefficients (model.py:200-202,216 in .eval()):
    alpha = fp32(w / sqrt(var + eps)) and beta = fp32(b - mean * alpha), each computed in
    fp64 from the fp32 parameters and rounded once."""
    w, b, m, v = (np.asarray(a, np.float32).astype(np.float64) for a in (weight, bias, running_mean, running_var))
    alpha = (w / np.sqrt(v + float(eps))).astype(np.float32)
    beta = (b - m * alpha.astype(np.float64)).astype(np.float32)
    return np.ascontiguousarray(alpha), np.ascontiguousarray(beta)


def query_proj(x, Wq, bq, alpha, beta, dt: str):
    """x [n, d], Wq [H, dq, d], bq [H, dq] (storage convention) -> q [n, H, dq]."""
    n, d = x.shape
    H, dq, _ = Wq.shape
    x, Wq, bq = (np.ascontiguousarray(a) for a in (x, Wq, bq))
    alpha = np.ascontiguousarray(alpha, np.float32).reshape(H, dq)
    beta = np.ascontiguousarray(beta, np.float32).reshape(H, dq)
    out = np.empty((n, H, dq), dtype=x.dtype)
    lib().ethos_oracle_query_proj(_p(x), _p(Wq), _p(bq), _p(alpha), _p(beta), n, d, H, dq, DT_CODE[dt], _p(out))
    return out


def subkey_scores(q, keys, half: int, dt: str):
    """q [rows, dq], keys [K, dq/2] -> float32 [rows, K] of T-rounded scores."""
    q = np.ascontiguousarray(q).reshape(-1, q.shape[-1])
    keys = np.ascontiguousarray(keys)
    rows, dq = q.shape
    K = keys.shape[0]
    out = np.empty((rows, K), np.float32)
    lib().ethos_oracle_subkey_scores(_p(q), _p(keys), rows, dq, half, K, DT_CODE[dt], _p(out))
    return out


def route(q, K1, K2, top_k: int, dt: str, k_cand: int | None = None, want_cand: bool = False):
    """q [..., dq] -> (gates [..., top_k] storage, ids [..., top_k] int32)."""
    lead = q.shape[:-1]
    dq = q.shape[-1]
    qf = np.ascontiguousarray(q).reshape(-1, dq)
    rows = qf.shape[0]
    K = K1.shape[0]
    kc = 2 * top_k if k_cand is None else k_cand
    gates = np.empty((rows, top_k), dtype=q.dtype)
    ids = np.empty((rows, top_k), dtype=np.int32)
    cand = np.empty((rows, 2, kc), dtype=np.int32) if want_cand else None
    rc = lib().ethos_oracle_route(_p(qf), _p(np.ascontiguousarray(K1)), _p(np.ascontiguousarray(K2)), rows, dq, K,
                                  top_k, kc, DT_CODE[dt], _p(gates), _p(ids),
                                  _p(cand) if want_cand else None)
    if rc != 0:
        raise ValueError(f"oracle route rejected sizes (rc={rc}): K={K} top_k={top_k} k_cand={kc}")
    out = (gates.reshape(*lead, top_k), ids.reshape(*lead, top_k))
    return out + (cand.reshape(*lead, 2, kc),) if want_cand else out


def select(s1, s2, top_k: int, dt: str, k_cand: int | None = None, want_cand: bool = False):
    """Selection stage from given T-valued score matrices s1, s2 [..., K] (float32)."""
    lead = s1.shape[:-1]
    K = s1.shape[-1]
    a = np.ascontiguousarray(s1, np.float32).reshape(-1, K)
    b = np.ascontiguousarray(s2, np.float32).reshape(-1, K)
    rows = a.shape[0]
    kc = 2 * top_k if k_cand is None else k_cand
    gates = np.empty((rows, top_k), dtype=np.uint16 if dt == "bf16" else np.float32)
    ids = np.empty((rows, top_k), dtype=np.int32)
    cand = np.empty((rows, 2, kc), dtype=np.int32) if want_cand else None
    rc = lib().ethos_oracle_select(_p(a), _p(b), rows, K, top_k, kc, DT_CODE[dt], _p(gates), _p(ids),
                                   _p(cand) if want_cand else None)
    if rc != 0:
        raise ValueError(f"oracle select rejected sizes (rc={rc})")
    out = (gates.reshape(*lead, top_k), ids.reshape(*lead, top_k))
    return out + (cand.reshape(*lead, 2, kc),) if want_cand else out


def sort_segment(ids, n_experts: int):
    """ids [n_pairs] -> (perm, uniq, seg_off, pair_slot); stable by pair index."""
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
    n = ids.shape[0]
    perm = np.empty(n, np.int32)
    uniq = np.empty(max(min(n, n_experts), 1), np.int32)
    seg = np.empty(max(min(n, n_experts), 1) + 1, np.int32)
    inv = np.empty(n, np.int32)
    U = lib().ethos_oracle_sort_segment(_p(ids), n, n_experts, _p(perm), _p(uniq), _p(seg), _p(inv))
    if U < 0:
        raise ValueError("expert id out of range")
    return perm, uniq[:U].copy(), seg[: U + 1].copy(), inv


# ------------------------------------------------------------------ generator / apply
def generate(latents, uniq, W1, W2, dt: str):
    """(h_e, v_e) for each expert id in ``uniq`` (model.py:168-179, 297-300, 320-323, 332).

    Rounding points mirror the reference's dtype flow: the pre-activation z W1 is
    rounded to T (a dtype matmul), GELU's output h is rounded to T, and v = h W_v
    (W_v = W2[d_model:]^T, model.py:300) is rounded to T.  Returns float32 arrays
    h [U, d_hidden] and v [U, d_model] holding T values.
    """
    d = W2.shape[0] // 2
    z = to_f32(latents[uniq], dt).astype(np.float64)
    w1 = to_f32(W1, dt).astype(np.float64)
    wv = to_f32(W2[d:], dt).astype(np.float64)
    pre = round_T(z @ w1.T, dt).astype(np.float64)
    hid = round_T(gelu64(pre), dt)
    return hid, round_T(hid.astype(np.float64) @ wv.T, dt)


def token_proj(x, W2, dt: str):
    """x_proj = RN_T(x W_u) [n_tok, d_hidden], W_u = W2[:d_model]^T (model.py:299, 326).

    The reference forms it inside the pair loop; it depends only on the token.
    """
    d = x.shape[1]
    xs = to_f32(x, dt).astype(np.float64)
    wu = to_f32(W2[:d], dt).astype(np.float64)                          # [d, d_hidden]
    return round_T(xs @ wu, dt)


def apply(xp, h, v, pair_slot, gates, n_heads: int, top_k: int, dt: str, tokens=None):
    """Weighted scatter-back (model.py:326-341) for the listed tokens (default all).

    Per pair p = (t, head, j) with expert slot s: a_p = RN(RN(gelu(RN(h_s . xp_t))) * g_p);
    per head y = RN(sum_j RN(a_p * v_s)) with the sum in high precision; the heads are
    summed in T one at a time and the result divided by H in T.  ``xp`` is
    token_proj(x).  Returns float32 [len(tokens), d] holding T values.
    """
    xpf = np.asarray(xp, np.float32)
    n_tok = xpf.shape[0]
    d = v.shape[1]
    g = to_f32(gates, dt).reshape(n_tok, n_heads, top_k)
    slot = np.asarray(pair_slot).reshape(n_tok, n_heads, top_k)
    toks = np.arange(n_tok) if tokens is None else np.asarray(tokens)
    hh = np.asarray(h).astype(np.float64)
    vv = np.asarray(v).astype(np.float64)
    out = np.empty((len(toks), d), np.float32)
    for i0 in range(0, len(toks), 32):
        tk = toks[i0:i0 + 32]
        xs = xpf[tk].astype(np.float64)                                 # [b, d_hidden]
        s = slot[tk]                                                      # [b, H, k]
        dots = np.einsum("bj,bhkj->bhk", xs, hh[s])                     # h_s . xp_t
        act = round_T(gelu64(round_T(dots, dt).astype(np.float64)), dt)
        a = round_T((act * g[tk]).astype(np.float32), dt)               # T * T product
        contrib = round_T((a[..., None].astype(np.float64) * vv[s]), dt)  # RN(a * v)
        head = round_T(contrib.astype(np.float64).sum(axis=2), dt)       # [b, H, d]
        acc = np.zeros((len(tk), d), np.float32)
        for hd in range(n_heads):
            acc = round_T((acc + head[:, hd]).astype(np.float32), dt)
        out[i0:i0 + len(tk)] = round_T((acc / np.float32(n_heads)).astype(np.float32), dt)
    return out


def apply_hidden(xp, h, W2, pair_slot, gates, n_heads: int, top_k: int, dt: str, tokens=None,
                 hacc_round: str = "T"):
    """Hidden-space reordering (paper/ETHOS.pdf p.10, Algorithm 1): per token
    h_acc = sum over the token's pairs of a_p h_s, then y = h_acc W_v, projected back once.

    Per pair p = (t, head, j) with expert slot s, a_p is the activation of ``apply``
    (RN(RN(gelu(RN(h_s . xp_t))) * g_p)).  h_acc sums RN32(a_p h_s) over heads, then j, in
    float32, scaled by 1/H (the layer's head average, model.py:341).  ``hacc_round``
    rounds h_acc / H before the projection: "T" to the layer dtype, "none" keeps float32.
    y = RN_T((h_acc / H) W_v) with an exact product (W_v = W2[d:]^T).  v rows never exist.
    Returns float32 [len(tokens), d] holding T values."""
    xpf = np.asarray(xp, np.float32)
    n_tok = xpf.shape[0]
    W2f = to_f32(W2, dt) if np.asarray(W2).dtype == np.uint16 else np.asarray(W2, np.float32)
    d = W2f.shape[0] // 2
    Wv = W2f[d:].astype(np.float64)                                      # [d, d_hidden]
    g = to_f32(gates, dt).reshape(n_tok, n_heads, top_k)
    slot = np.asarray(pair_slot).reshape(n_tok, n_heads, top_k)
    toks = np.arange(n_tok) if tokens is None else np.asarray(tokens)
    hh = np.asarray(h).astype(np.float64)
    hf32 = np.asarray(h, np.float32)
    out = np.empty((len(toks), d), np.float32)
    for i0 in range(0, len(toks), 32):
        tk = toks[i0:i0 + 32]
        xs = xpf[tk].astype(np.float64)
        s = slot[tk]
        dots = np.einsum("bj,bhkj->bhk", xs, hh[s])
        act = round_T(gelu64(round_T(dots, dt).astype(np.float64)), dt)
        a = round_T((act * g[tk]).astype(np.float32), dt).astype(np.float32)
        acc = np.zeros((len(tk), hh.shape[1]), np.float32)
        for hd in range(n_heads):
            for j in range(top_k):
                acc = (acc + (a[:, hd, j, None] * hf32[s[:, hd, j]]).astype(np.float32)).astype(np.float32)
        acc = (acc / np.float32(n_heads)).astype(np.float32)
        if hacc_round == "T":
            acc = round_T(acc, dt).astype(np.float32)
        out[i0:i0 + len(tk)] = round_T(acc.astype(np.float64) @ Wv.T, dt)
    return out


# ------------------------------------------------------------------ whole layer
def unpack_state(sd: dict, H: int):
    """Reference state_dict (torch CPU tensors) -> numpy arrays in storage convention."""
    import torch

    Wq = torch.stack([sd[f"router.query_projs.{h}.weight"] for h in range(H)])
    bq = torch.stack([sd[f"router.query_projs.{h}.bias"] for h in range(H)])
    bn = [
        bn_coeffs(*(sd[f"router.query_norms.{h}.{n}"].float().numpy() for n in ("weight", "bias", "running_mean", "running_var")))
        for h in range(H)
    ]
    return dict(
        latents=from_torch(sd["expert_latents.weight"]),
        W1=from_torch(sd["generation_network.net.0.weight"]),
        W2=from_torch(sd["generation_network.net.2.weight"]),
        Wq=from_torch(Wq),
        bq=from_torch(bq),
        alpha=np.stack([a for a, _ in bn]).astype(np.float32),
        beta=np.stack([b for _, b in bn]).astype(np.float32),
        K1=from_torch(sd["router.sub_keys_1.weight"]),
        K2=from_torch(sd["router.sub_keys_2.weight"]),
    )


def layer_forward(x, P: dict, n_heads: int, top_k: int, dt: str, tokens=None, q=None, routed=None):
    """Full expert-layer forward; returns a dict of every intermediate.

    ``tokens`` restricts the generator and apply stages to those tokens (routing
    still covers every token).  ``q`` skips the projection with a given query;
    ``routed`` = (gates, ids), this function's own routing of that query computed
    earlier, skips the routing as well.
    """
    if q is None:
        q = query_proj(x, P["Wq"], P["bq"], P["alpha"], P["beta"], dt)
    gates, ids = route(q, P["K1"], P["K2"], top_k, dt) if routed is None else routed
    n_tok = x.shape[0]
    E = P["latents"].shape[0]
    sel_ids = ids if tokens is None else ids[np.asarray(tokens)]
    perm, uniq, seg, inv = sort_segment(ids.reshape(-1), E)
    xp = token_proj(x, P["W2"], dt)
    if tokens is None:
        h, v = generate(P["latents"], uniq, P["W1"], P["W2"], dt)
        out = apply(xp, h, v, inv, gates, n_heads, top_k, dt)
    else:
        # generate only the experts the listed tokens use; remap slots
        sub_uniq = np.unique(sel_ids.reshape(-1))
        h_sub, v_sub = generate(P["latents"], sub_uniq, P["W1"], P["W2"], dt)
        full_slot = np.searchsorted(sub_uniq, ids.reshape(-1)).clip(0, len(sub_uniq) - 1)
        out = apply(xp, h_sub, v_sub, full_slot, gates, n_heads, top_k, dt, tokens=tokens)
        h = v = None
    return dict(q=q, gates=gates, ids=ids, perm=perm, uniq=uniq, seg_off=seg, pair_slot=inv, xp=xp, h=h, v=v,
                out=out)
