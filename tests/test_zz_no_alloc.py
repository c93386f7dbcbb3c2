"""ethos_sort_segment_noalloc (the sort without a caller workspace) against
ethos_sort_segment through the C-ABI: bit-identical outputs on three calls in a row, each
with fewer pairs than the last.  The second (300,000 pairs, another id mix) takes the
tiled path over the static workspace that still holds the first call's data; the third
(5,000 pairs) the single-workgroup sort, which does not use the static workspace."""
import numpy as np
import pytest
import torch

from ethos_amd import _lib, hip
from oracle import oracle as O

pytestmark = pytest.mark.gpu

E = 262144


def _outputs(n, dev):
    max_u = max(1, min(n, E))
    # filled with a marker so that a missing write shows as a difference
    return dict(perm=torch.full((n,), -7, dtype=torch.int32, device=dev),
                uniq=torch.full((max_u,), -7, dtype=torch.int32, device=dev),
                seg_off=torch.full((max_u + 1,), -7, dtype=torch.int32, device=dev),
                pair_slot=torch.full((n,), -7, dtype=torch.int32, device=dev),
                sorted_slot=torch.full((n,), -7, dtype=torch.int32, device=dev),
                n_unique=torch.full((1,), -7, dtype=torch.int32, device=dev))


def _with_workspace(ids):
    L = _lib.load()
    n = ids.numel()
    r = _outputs(n, ids.device)
    ws, ws_bytes = hip.workspace(L.ethos_sort_workspace_bytes(n, E), ids.device)
    rc = L.ethos_sort_segment(ids.data_ptr(), n, E, ws.data_ptr(), ws_bytes, r["perm"].data_ptr(),
                              r["uniq"].data_ptr(), r["seg_off"].data_ptr(), r["pair_slot"].data_ptr(),
                              r["sorted_slot"].data_ptr(), r["n_unique"].data_ptr(),
                              torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "ethos_sort_segment")
    return r


def _no_alloc(ids):
    L = _lib.load()
    n = ids.numel()
    r = _outputs(n, ids.device)
    rc = L.ethos_sort_segment_noalloc(ids.data_ptr(), n, E, r["perm"].data_ptr(), r["uniq"].data_ptr(),
                                      r["seg_off"].data_ptr(), r["pair_slot"].data_ptr(),
                                      r["sorted_slot"].data_ptr(), r["n_unique"].data_ptr(),
                                      torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "ethos_sort_segment_noalloc")
    return r


def _ids(n, seed, hot_share=0.5, n_hot=300):
    """Uniform ids, with a share of the pairs drawn from a few hundred hot experts (long
    segments)."""
    g = torch.Generator().manual_seed(seed)
    nh = int(n * hot_share)
    uni = torch.randint(0, E, (n - nh,), generator=g)
    hot = torch.randint(0, n_hot, (nh,), generator=g) * (E // n_hot - 1)  # ids below E
    ids = torch.cat([uni, hot])[torch.randperm(n, generator=g)]
    return ids.to(torch.int32)


def _same(a, b):
    U = int(a["n_unique"].item())
    assert U == int(b["n_unique"].item())
    for k in ("perm", "pair_slot", "sorted_slot"):
        assert torch.equal(a[k], b[k]), k
    assert torch.equal(a["uniq"][:U], b["uniq"][:U])
    assert torch.equal(a["seg_off"][: U + 1], b["seg_off"][: U + 1])
    return U


def test_sort_noalloc_matches_sort_with_workspace():
    dev = torch.device("cuda")
    for n, seed, share, n_hot in ((_lib.NOALLOC_MAX_PAIRS, 1, 0.5, 300), (300000, 3, 0.8, 40), (5000, 2, 0.5, 300)):
        print(f"sort_noalloc: {n} pairs, seed {seed}", flush=True)
        ids = _ids(n, seed, share, n_hot)
        want = _with_workspace(ids.to(dev))
        got = _no_alloc(ids.to(dev))
        torch.cuda.synchronize()
        U = _same(got, want)
        # and the sort itself against the oracle's stable counting sort
        perm, uniq, seg, inv = O.sort_segment(ids.numpy(), E)
        assert np.array_equal(got["perm"].cpu().numpy(), perm)
        assert np.array_equal(got["uniq"][:U].cpu().numpy(), uniq)
        assert np.array_equal(got["seg_off"][: U + 1].cpu().numpy(), seg)
        assert np.array_equal(got["pair_slot"].cpu().numpy(), inv)


def test_sort_noalloc_empty_and_limit():
    dev = torch.device("cuda")
    r = _outputs(0, dev)
    L = _lib.load()
    rc = L.ethos_sort_segment_noalloc(None, 0, E, None, None, r["seg_off"].data_ptr(), None, None,
                                      r["n_unique"].data_ptr(), torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "ethos_sort_segment_noalloc")
    torch.cuda.synchronize()
    assert int(r["n_unique"].item()) == 0 and int(r["seg_off"][0].item()) == 0
    ids = torch.zeros(_lib.NOALLOC_MAX_PAIRS + 1, dtype=torch.int32, device=dev)
    rc = L.ethos_sort_segment_noalloc(ids.data_ptr(), ids.numel(), E, 16, 16, 16, 16, 16, 16, None)
    assert rc == -2
