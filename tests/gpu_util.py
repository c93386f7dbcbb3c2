"""Helpers shared by the GPU parity tests."""
import numpy as np
import torch

from oracle import oracle as O
from torch_reference import apply_from_routing


def to_dev(a: np.ndarray, dt: str | None = None) -> torch.Tensor:
    """numpy (oracle storage convention) -> device tensor."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).cuda()
    return torch.from_numpy(a).cuda()


def to_host(t: torch.Tensor) -> np.ndarray:
    return O.from_torch(t)


def state_to_dev(sd: dict) -> dict:
    return {k: v.cuda() for k, v in sd.items()}


def check_out(out: np.ndarray, ref: np.ndarray, dt: str, signal: bool = False, nerr_max: float = 1e-2):
    """Layer-output tolerance.  fp32: |d| <= 1e-4|ref| + 1e-4 max|ref|.  bf16: the stated
    rtol 2e-2 / atol 2e-3 (natural scale only), |d| <= 2e-2|ref| + 1e-2 max|ref|, and
    ||d|| / ||ref|| <= nerr_max."""
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.abs(out - ref)
    m = np.abs(ref).max() if ref.size else 0.0
    if dt == "fp32":
        bad = d > 1e-4 * np.abs(ref) + 1e-4 * m
        assert not bad.any(), f"{bad.sum()} fp32 elements out of tolerance, max |d| {d.max():.3e}, max|ref| {m:.3e}"
    else:
        if not signal:
            assert np.all(d <= 2e-2 * np.abs(ref) + 2e-3)
        bad = d > 2e-2 * np.abs(ref) + 1e-2 * m
        assert not bad.any(), f"{bad.sum()} bf16 elements out of tolerance, max |d|/max|ref| {(d / m).max():.3e}"
        nerr = np.linalg.norm(d) / max(np.linalg.norm(ref), 1e-30)
        assert nerr <= nerr_max, f"normalised error {nerr:.3e} > {nerr_max}"


# Every token's output against the float32 expert stages (model.py:312-341) on the same
# routing, measured against the size of the token's terms: the bf16 roundings of the
# contract stay below this; a dropped pair or a pair on the wrong expert is ~1/sqrt(H k).
ALL_TOKENS_BF16 = 2e-2


def check_all_tokens(m, x, gates, ids, y, label):
    with torch.no_grad():
        yr, scale = apply_from_routing(m.state_dict(), x, gates, ids, m.num_heads)
    err = (y.float() - yr).norm(dim=1) / scale.clamp_min(1e-3 * float(scale.max()))
    print(f"{label}: all {err.numel()} tokens against the float32 expert stages: error / term size "
          f"median {float(err.median()):.2e}, max {float(err.max()):.2e}", flush=True)
    assert bool(torch.isfinite(y).all()) and float(err.max()) < ALL_TOKENS_BF16
