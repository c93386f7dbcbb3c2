"""Torch-facing wrappers of the C-ABI: validate, allocate outputs from the caching
allocator, enqueue on the current stream.  Every function requires CUDA (HIP)
tensors and raises on anything else -- there is no CPU path.
"""
from __future__ import annotations

import torch

from ._lib import check, dtype_code, load


def _stream_slow() -> int:
    return torch.cuda.current_stream().cuda_stream


def _stream_fast() -> int:
    return torch._C._cuda_getCurrentRawStream(torch._C._cuda_getDevice())


# The current device's current stream as a hipStream_t; the raw accessor skips the Python
# device bookkeeping of torch.cuda.current_stream (a few microseconds per call).
_stream = _stream_fast if hasattr(torch._C, "_cuda_getCurrentRawStream") else _stream_slow


def _need(t: torch.Tensor, name: str, dtype=None, dim=None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be on a HIP device (got {t.device}); the ETHOS kernels have no CPU path")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if dim is not None and t.dim() != dim:
        raise RuntimeError(f"{name} must have {dim} dims, got shape {tuple(t.shape)}")


def workspace(nbytes: int, device) -> tuple[torch.Tensor, int]:
    """A scratch buffer of at least `nbytes` bytes (int64 storage keeps it 16-byte
    aligned) and its real size, which is what the ABI is told."""
    ws = torch.empty((max(1, (nbytes + 7) // 8),), dtype=torch.int64, device=device)
    size = ws.numel() * ws.element_size()
    if size < nbytes:
        raise AssertionError("workspace sizing")
    return ws, size


def stage_events(events) -> None:
    """Hand the library torch.cuda.Event objects (already recorded once, so that they exist)
    to record, in order, at the stage boundaries of this thread's next calls; [] clears."""
    import ctypes

    handles = [e.cuda_event for e in events]
    if any(h == 0 for h in handles):
        raise RuntimeError("stage_events: record each event once before handing it over")
    arr = (ctypes.c_void_p * max(1, len(handles)))(*handles)
    check(load().ethos_stage_events(arr, len(handles)), "ethos_stage_events")


def key_norm_bounds(sub_keys_1: torch.Tensor, sub_keys_2: torch.Tensor) -> torch.Tensor:
    """fp32 [2, K] upper bounds of the sub-key row norms: fp64 norms of the stored
    values, inflated by 2^-20 and rounded, on the host (once per parameter version)."""
    import numpy as np

    rows = []
    for t in (sub_keys_1, sub_keys_2):
        v = t.detach().float().cpu().numpy().astype(np.float64)
        rows.append((np.sqrt((v * v).sum(axis=1)) * (1.0 + 2.0 ** -20)).astype(np.float32))
    return torch.from_numpy(np.stack(rows)).contiguous()


def query_proj_prepare(wq: torch.Tensor) -> torch.Tensor | None:
    """The prepared form of wq [H, dq, d] for query_proj(..., prepared=...) (a uint8 device
    buffer), or None when the dtype has nothing to prepare (fp32)."""
    _need(wq, "wq", dim=3)
    H, dq, d = wq.shape
    n = load().ethos_query_proj_weights_bytes(d, H, dq, dtype_code(wq.dtype))
    if n == 0:
        return None
    buf = torch.empty(n, dtype=torch.uint8, device=wq.device)
    rc = load().ethos_query_proj_prepare(wq.data_ptr(), d, H, dq, dtype_code(wq.dtype), buf.data_ptr(), n, _stream())
    check(rc, "ethos_query_proj_prepare")
    return buf


def query_proj(x: torch.Tensor, wq: torch.Tensor, bq: torch.Tensor, bn_alpha: torch.Tensor, bn_beta: torch.Tensor,
               out: torch.Tensor | None = None, prepared: torch.Tensor | None = None) -> torch.Tensor:
    """x [n, d], wq [H, dq, d], bq [H, dq], bn_alpha/beta [H, dq] fp32 -> q [n, H, dq].
    prepared: query_proj_prepare(wq) of the same wq, or None."""
    _need(x, "x", dim=2)
    _need(wq, "wq", x.dtype, 3)
    _need(bq, "bq", x.dtype, 2)
    _need(bn_alpha, "bn_alpha", torch.float32)
    _need(bn_beta, "bn_beta", torch.float32)
    n, d = x.shape
    H, dq, d2 = wq.shape
    if d2 != d or bq.shape != (H, dq) or bn_alpha.numel() != H * dq or bn_beta.numel() != H * dq:
        raise RuntimeError("query_proj: inconsistent shapes")
    if out is None:
        out = torch.empty((n, H, dq), dtype=x.dtype, device=x.device)
    ws, ws_bytes = workspace(load().ethos_query_proj_workspace_bytes(n, d, H, dq, dtype_code(x.dtype)), x.device)
    if prepared is not None:
        _need(prepared, "prepared", torch.uint8, 1)
        rc = load().ethos_query_proj_prepared(x.data_ptr(), wq.data_ptr(), prepared.data_ptr(), prepared.numel(),
                                              bq.data_ptr(),
                                              bn_alpha.data_ptr(), bn_beta.data_ptr(), n, d, H, dq,
                                              dtype_code(x.dtype), ws.data_ptr(), ws_bytes, out.data_ptr(), _stream())
        check(rc, "ethos_query_proj_prepared")
        return out
    rc = load().ethos_query_proj(x.data_ptr(), wq.data_ptr(), bq.data_ptr(), bn_alpha.data_ptr(), bn_beta.data_ptr(),
                                 n, d, H, dq, dtype_code(x.dtype), ws.data_ptr(), ws_bytes, out.data_ptr(), _stream())
    check(rc, "ethos_query_proj")
    return out


def route_prepare_keys(sub_keys_1: torch.Tensor, sub_keys_2: torch.Tensor) -> torch.Tensor:
    """Both sub-key tables [K, dq/2] in the scoring MFMAs' fragment order (a uint8 device
    buffer) for route_topk(..., prepared_keys=...)."""
    _need(sub_keys_1, "sub_keys_1", dim=2)
    _need(sub_keys_2, "sub_keys_2", sub_keys_1.dtype, 2)
    K, dh2 = sub_keys_1.shape
    if sub_keys_2.shape != (K, dh2):
        raise RuntimeError("route_prepare_keys: the two sub-key tables must have the same shape")
    code = dtype_code(sub_keys_1.dtype)
    n = load().ethos_route_keys_bytes(K, 2 * dh2, code)
    if n == 0:
        raise RuntimeError(f"route_prepare_keys: unsupported sub-key tables {tuple(sub_keys_1.shape)}")
    buf = torch.empty(n, dtype=torch.uint8, device=sub_keys_1.device)
    rc = load().ethos_route_prepare_keys(sub_keys_1.data_ptr(), sub_keys_2.data_ptr(), K, 2 * dh2, code,
                                         buf.data_ptr(), n, _stream())
    check(rc, "ethos_route_prepare_keys")
    return buf


def route_topk(q: torch.Tensor, sub_keys_1: torch.Tensor, sub_keys_2: torch.Tensor, top_k: int,
               k_cand: int | None = None, key_norms: torch.Tensor | None = None,
               prepared_keys: torch.Tensor | None = None):
    """q [..., dq] -> (gates [..., top_k] q.dtype, expert ids [..., top_k] int32).
    key_norms: optional fp32 [2, K] upper bounds of the sub-key row norms; prepared_keys:
    optional route_prepare_keys(sub_keys_1, sub_keys_2) (the same results, faster)."""
    _need(q, "q")
    _need(sub_keys_1, "sub_keys_1", q.dtype, 2)
    _need(sub_keys_2, "sub_keys_2", q.dtype, 2)
    dq = q.shape[-1]
    K = sub_keys_1.shape[0]
    if sub_keys_1.shape != (K, dq // 2) or sub_keys_2.shape != (K, dq // 2):
        raise RuntimeError("route_topk: sub-key tables must be [K, d_query/2]")
    kc = 2 * top_k if k_cand is None else k_cand
    rows = q.numel() // dq
    gates = torch.empty((*q.shape[:-1], top_k), dtype=q.dtype, device=q.device)
    ids = torch.empty((*q.shape[:-1], top_k), dtype=torch.int32, device=q.device)
    if key_norms is not None:
        _need(key_norms, "key_norms", torch.float32)
        if key_norms.numel() != 2 * K:
            raise RuntimeError("route_topk: key_norms must hold 2 * K values")
    kn = key_norms.data_ptr() if key_norms is not None else None
    if prepared_keys is not None:
        _need(prepared_keys, "prepared_keys", torch.uint8)
        rc = load().ethos_route_topk_prepared(q.data_ptr(), sub_keys_1.data_ptr(), sub_keys_2.data_ptr(), kn,
                                              prepared_keys.data_ptr(), prepared_keys.numel(), rows, dq, K, top_k, kc,
                                              dtype_code(q.dtype), gates.data_ptr(), ids.data_ptr(), _stream())
        check(rc, "ethos_route_topk_prepared")
    else:
        rc = load().ethos_route_topk(q.data_ptr(), sub_keys_1.data_ptr(), sub_keys_2.data_ptr(), kn, rows, dq, K,
                                     top_k, kc, dtype_code(q.dtype), gates.data_ptr(), ids.data_ptr(), _stream())
        check(rc, "ethos_route_topk")
    return gates, ids


def sort_segment(ids: torch.Tensor, n_experts: int) -> dict:
    """Reorder pairs by expert id.  Returns perm, uniq, seg_off, pair_slot, sorted_slot,
    n_unique (device int32[1]) and max_unique (host int, the buffer bound)."""
    _need(ids, "ids", torch.int32)
    n = ids.numel()
    dev = ids.device
    max_u = max(1, min(n, n_experts))
    ws, ws_bytes = workspace(load().ethos_sort_workspace_bytes(n, n_experts), dev)
    r = dict(
        perm=torch.empty(n, dtype=torch.int32, device=dev),
        uniq=torch.empty(max_u, dtype=torch.int32, device=dev),
        seg_off=torch.empty(max_u + 1, dtype=torch.int32, device=dev),
        pair_slot=torch.empty(n, dtype=torch.int32, device=dev),
        sorted_slot=torch.empty(n, dtype=torch.int32, device=dev),
        n_unique=torch.empty(1, dtype=torch.int32, device=dev),
        max_unique=max_u,
    )
    rc = load().ethos_sort_segment(ids.data_ptr(), n, n_experts, ws.data_ptr(), ws_bytes, r["perm"].data_ptr(),
                                   r["uniq"].data_ptr(), r["seg_off"].data_ptr(), r["pair_slot"].data_ptr(),
                                   r["sorted_slot"].data_ptr(), r["n_unique"].data_ptr(), _stream())
    check(rc, "ethos_sort_segment")
    return r


# Pairs up to which the sort runs as one workgroup (and ethos_sort_segment_token_proj runs the
# bf16 token projection in the same launch).
SMALL_SORT_MAX = 16384


def sort_segment_token_proj(ids: torch.Tensor, n_experts: int, x: torch.Tensor, w2: torch.Tensor,
                            wut: torch.Tensor | None) -> tuple[dict, torch.Tensor]:
    """sort_segment(ids, n_experts) and token_proj(x, w2, wut) in one library call: one
    launch for bf16 batches of at most SMALL_SORT_MAX pairs with wut given, the two in turn
    otherwise.  Returns (the sort's dict, x_proj)."""
    _need(ids, "ids", torch.int32)
    _need(x, "x", dim=2)
    _need(w2, "w2", x.dtype, 2)
    n = ids.numel()
    dev = ids.device
    n_tok, d = x.shape
    dh = w2.shape[1]
    if w2.shape[0] != 2 * d:
        raise RuntimeError("sort_segment_token_proj: w2 must be [2 d_model, d_hidden]")
    if wut is not None:
        _need(wut, "wut", x.dtype, 2)
        if wut.shape != (dh, d):
            raise RuntimeError("sort_segment_token_proj: wut must be [d_hidden, d_model]")
    max_u = max(1, min(n, n_experts))
    ws, ws_bytes = workspace(load().ethos_sort_workspace_bytes(n, n_experts), dev)
    r = dict(
        perm=torch.empty(n, dtype=torch.int32, device=dev),
        uniq=torch.empty(max_u, dtype=torch.int32, device=dev),
        seg_off=torch.empty(max_u + 1, dtype=torch.int32, device=dev),
        pair_slot=torch.empty(n, dtype=torch.int32, device=dev),
        sorted_slot=torch.empty(n, dtype=torch.int32, device=dev),
        n_unique=torch.empty(1, dtype=torch.int32, device=dev),
        max_unique=max_u,
    )
    xp = torch.empty((n_tok, dh), dtype=x.dtype, device=x.device)
    rc = load().ethos_sort_segment_token_proj(
        ids.data_ptr(), n, n_experts, ws.data_ptr(), ws_bytes, r["perm"].data_ptr(), r["uniq"].data_ptr(),
        r["seg_off"].data_ptr(), r["pair_slot"].data_ptr(), r["sorted_slot"].data_ptr(), r["n_unique"].data_ptr(),
        x.data_ptr(), w2.data_ptr(), wut.data_ptr() if wut is not None else None, n_tok, d, dh, dtype_code(x.dtype),
        xp.data_ptr(), _stream())
    check(rc, "ethos_sort_segment_token_proj")
    return r, xp


def generate(latents: torch.Tensor, uniq: torch.Tensor, n_unique: torch.Tensor, max_unique: int, w1: torch.Tensor,
             w2: torch.Tensor, with_v: bool = True) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Hidden rows h [max_unique, d_hidden] and v rows [max_unique, d] of the unique experts
    (rows >= U unspecified).  with_v=False produces h only (v is None), as the
    hidden-space apply needs."""
    _need(latents, "latents", dim=2)
    _need(uniq, "uniq", torch.int32)
    _need(n_unique, "n_unique", torch.int32)
    _need(w1, "w1", latents.dtype, 2)
    _need(w2, "w2", latents.dtype, 2)
    E, dl = latents.shape
    dh = w1.shape[0]
    if w1.shape != (dh, dl) or w2.shape[1] != dh or w2.shape[0] % 2:
        raise RuntimeError("generate: inconsistent weight shapes")
    d = w2.shape[0] // 2
    h = torch.empty((max_unique, dh), dtype=latents.dtype, device=latents.device)
    v = torch.empty((max_unique, d), dtype=latents.dtype, device=latents.device) if with_v else None
    rc = load().ethos_generate(latents.data_ptr(), E, uniq.data_ptr(), n_unique.data_ptr(), max_unique, w1.data_ptr(),
                               w2.data_ptr(), dl, dh, d, dtype_code(latents.dtype), h.data_ptr(),
                               v.data_ptr() if with_v else None, _stream())
    check(rc, "ethos_generate")
    return h, v


def apply_scatter(x: torch.Tensor, w2: torch.Tensor, h: torch.Tensor, v: torch.Tensor, seg: dict,
                  gates: torch.Tensor, n_heads: int, top_k: int) -> torch.Tensor:
    """out [n, d] = head-averaged weighted sum of the experts' contributions."""
    _need(x, "x", dim=2)
    _need(w2, "w2", x.dtype, 2)
    _need(h, "h", x.dtype, 2)
    _need(v, "v", x.dtype, 2)
    _need(gates, "gates", x.dtype)
    n, d = x.shape
    dh = h.shape[1]
    if w2.shape != (2 * d, dh) or v.shape[1] != d or gates.numel() != n * n_heads * top_k:
        raise RuntimeError("apply_scatter: inconsistent shapes")
    code = dtype_code(x.dtype)
    ws, ws_bytes = workspace(load().ethos_apply_workspace_bytes(n, n_heads, top_k, dh, code), x.device)
    out = torch.empty_like(x)
    rc = load().ethos_apply_scatter(x.data_ptr(), w2.data_ptr(), h.data_ptr(), v.data_ptr(), seg["perm"].data_ptr(),
                                    seg["sorted_slot"].data_ptr(), seg["pair_slot"].data_ptr(), gates.data_ptr(), n,
                                    n_heads, top_k, d, dh, code, ws.data_ptr(), ws_bytes, out.data_ptr(), _stream())
    check(rc, "ethos_apply_scatter")
    return out


def apply_hidden(x: torch.Tensor, w2: torch.Tensor, h: torch.Tensor, seg: dict, gates: torch.Tensor, n_heads: int,
                 top_k: int) -> torch.Tensor:
    """out [n, d] by hidden-space reordering: per token (1/H) sum_p a_p h_s, projected by W_v
    once (no v rows)."""
    _need(x, "x", dim=2)
    _need(w2, "w2", x.dtype, 2)
    _need(h, "h", x.dtype, 2)
    _need(gates, "gates", x.dtype)
    n, d = x.shape
    dh = h.shape[1]
    if w2.shape != (2 * d, dh) or gates.numel() != n * n_heads * top_k:
        raise RuntimeError("apply_hidden: inconsistent shapes")
    code = dtype_code(x.dtype)
    ws, ws_bytes = workspace(load().ethos_apply_hidden_workspace_bytes(n, n_heads, top_k, d, dh, code), x.device)
    out = torch.empty_like(x)
    rc = load().ethos_apply_hidden(x.data_ptr(), w2.data_ptr(), h.data_ptr(), seg["perm"].data_ptr(),
                                   seg["sorted_slot"].data_ptr(), seg["pair_slot"].data_ptr(), gates.data_ptr(), n,
                                   n_heads, top_k, d, dh, code, ws.data_ptr(), ws_bytes, out.data_ptr(), _stream())
    check(rc, "ethos_apply_hidden")
    return out


def token_proj(x: torch.Tensor, w2: torch.Tensor, wut: torch.Tensor | None = None,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """x_proj [n, d_hidden] = RN(x W_u), W_u = w2[:d] ([d, d_hidden]); bf16 needs wut = W_u^T
    ([d_hidden, d]) for d % 64 == 0.  `out`: optional [n, d_hidden] destination."""
    _need(x, "x", dim=2)
    _need(w2, "w2", x.dtype, 2)
    n, d = x.shape
    dh = w2.shape[1]
    if w2.shape[0] != 2 * d:
        raise RuntimeError("token_proj: w2 must be [2 d_model, d_hidden]")
    if wut is not None:
        _need(wut, "wut", x.dtype, 2)
        if wut.shape != (dh, d):
            raise RuntimeError("token_proj: wut must be [d_hidden, d_model]")
    if out is not None:
        _need(out, "out", x.dtype, 2)
        if out.shape != (n, dh):
            raise RuntimeError("token_proj: out must be [n_tok, d_hidden]")
    xp = torch.empty((n, dh), dtype=x.dtype, device=x.device) if out is None else out
    rc = load().ethos_token_proj(x.data_ptr(), w2.data_ptr(), wut.data_ptr() if wut is not None else None, n, d, dh,
                                 dtype_code(x.dtype), xp.data_ptr(), _stream())
    check(rc, "ethos_token_proj")
    return xp


def expert_forward(x: torch.Tensor, latents: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, seg: dict,
                   gates: torch.Tensor, n_heads: int, top_k: int, hidden_space: bool = False,
                   wut: torch.Tensor | None = None, xp: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(out [n, d], h [max_unique, d_hidden]): generation, activations and scatter-back
    (or, hidden_space=True, the hidden-space form) in one call.  `wut`: optional bf16
    W_u^T [d_hidden, d] (the transpose of w2[:d]) prepared by the caller; `xp`: optional
    token projection from token_proj (then not recomputed)."""
    _need(x, "x", dim=2)
    _need(latents, "latents", x.dtype, 2)
    _need(w1, "w1", x.dtype, 2)
    _need(w2, "w2", x.dtype, 2)
    _need(gates, "gates", x.dtype)
    n, d = x.shape
    E, dl = latents.shape
    dh = w1.shape[0]
    if w1.shape != (dh, dl) or w2.shape != (2 * d, dh) or gates.numel() != n * n_heads * top_k:
        raise RuntimeError("expert_forward: inconsistent shapes")
    if wut is not None:
        _need(wut, "wut", x.dtype, 2)
        if wut.shape != (dh, d):
            raise RuntimeError("expert_forward: wut must be [d_hidden, d_model]")
    if xp is not None:
        _need(xp, "xp", x.dtype, 2)
        if xp.shape != (n, dh):
            raise RuntimeError("expert_forward: xp must be [n_tok, d_hidden]")
    code = dtype_code(x.dtype)
    order = 1 if hidden_space else 0
    max_u = seg["max_unique"]
    ws, ws_bytes = workspace(load().ethos_expert_forward_workspace_bytes(n, n_heads, top_k, max_u, d, dh, code, order),
                             x.device)
    h = torch.empty((max_u, dh), dtype=x.dtype, device=x.device)
    out = torch.empty_like(x)
    rc = load().ethos_expert_forward(x.data_ptr(), latents.data_ptr(), E, w1.data_ptr(), w2.data_ptr(),
                                     wut.data_ptr() if wut is not None else None,
                                     xp.data_ptr() if xp is not None else None, seg["uniq"].data_ptr(),
                                     seg["seg_off"].data_ptr(), seg["n_unique"].data_ptr(), max_u, seg["perm"].data_ptr(),
                                     seg["sorted_slot"].data_ptr(), seg["pair_slot"].data_ptr(), gates.data_ptr(), n,
                                     n_heads, top_k, dl, dh, d, code, order, ws.data_ptr(), ws_bytes, h.data_ptr(),
                                     out.data_ptr(), _stream())
    check(rc, "ethos_expert_forward")
    return out, h


def expert_backward(h: torch.Tensor, xp: torch.Tensor, dyb: torch.Tensor, seg: dict, gates: torch.Tensor,
                    n_heads: int, top_k: int, U: int):
    """Per-pair part of the expert stages' backward: (dgates [n, H, k], hacc [n, dh], dxp [n, dh],
    dh [U, dh]), all float32, from xp = x W_u and dyb = (dy / H) W_v^T (float32 [n, dh]) and the
    routing's sorted segments `seg` (sort_segment); deterministic (fixed summation orders)."""
    _need(h, "h", dim=2)
    _need(xp, "xp", torch.float32, 2)
    _need(dyb, "dyb", torch.float32, 2)
    pair_slot = seg["pair_slot"]
    _need(pair_slot, "pair_slot", torch.int32)
    _need(gates, "gates", h.dtype)
    n, dh = xp.shape
    if dyb.shape != (n, dh) or h.shape[1] != dh or gates.numel() != n * n_heads * top_k:
        raise RuntimeError("expert_backward: inconsistent shapes")
    dev = h.device
    dg = torch.empty(gates.shape, dtype=torch.float32, device=dev)
    hacc = torch.empty((n, dh), dtype=torch.float32, device=dev)
    dxp = torch.empty((n, dh), dtype=torch.float32, device=dev)
    dhs = torch.empty((max(U, 1), dh), dtype=torch.float32, device=dev)
    ws, ws_bytes = workspace(load().ethos_expert_backward_workspace_bytes(n, n_heads, top_k, dh), dev)
    rc = load().ethos_expert_backward(h.data_ptr(), xp.data_ptr(), dyb.data_ptr(), pair_slot.data_ptr(),
                                      seg["perm"].data_ptr(), seg["sorted_slot"].data_ptr(), seg["seg_off"].data_ptr(),
                                      gates.data_ptr(), n, n_heads, top_k, dh, dtype_code(h.dtype), ws.data_ptr(),
                                      ws_bytes, dg.data_ptr(), hacc.data_ptr(), dxp.data_ptr(), dhs.data_ptr(),
                                      _stream())
    check(rc, "ethos_expert_backward")
    return dg, hacc, dxp, dhs[:U]
