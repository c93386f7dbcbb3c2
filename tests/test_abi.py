"""The C-ABI library loads and exports every entry point include/ethos_hip.h declares;
argument errors come back as codes (checked without a GPU: validation runs before
any HIP call)."""
import ctypes
import os
import re

import pytest

from ethos_amd import _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "ethos_hip.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(ethos_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    assert names == sorted(_lib.SIGNATURES), names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_abi_version():
    assert _lib.load().ethos_abi_version() == 8


def _rc(fn, *args):
    return getattr(_lib.load(), fn)(*args)


def test_argument_errors_are_codes():
    L = _lib.load()
    # unknown dtype
    assert L.ethos_route_topk(16, 16, 16, None, 4, 32, 16, 2, 4, 7, 16, 16, None) == -1
    assert b"dtype" in L.ethos_last_error()
    # k_cand larger than the sub-key count (the reference's torch.topk would raise)
    assert L.ethos_route_topk(16, 16, 16, None, 4, 32, 16, 16, 32, 1, 16, 16, None) == -2
    # k_cand beyond this build's limit
    assert L.ethos_route_topk(16, 16, 16, None, 4, 32, 4096, 32, 64, 1, 16, 16, None) == -6
    # odd d_query
    assert L.ethos_route_topk(16, 16, 16, None, 4, 7, 16, 2, 4, 1, 16, 16, None) == -2
    # null pointers
    assert L.ethos_query_proj(None, 16, 16, 16, 16, 4, 8, 2, 8, 1, 16, 4096, 16, None) == -3
    # bf16 needs its workspace
    assert L.ethos_query_proj(16, 16, 16, 16, 16, 4, 64, 2, 8, 1, 16, 8, 16, None) == -5
    # prepared weights: missing, or smaller than their size (bf16); fp32 has nothing to prepare
    need = L.ethos_query_proj_weights_bytes(64, 2, 8, 1)
    assert need > 0 and L.ethos_query_proj_weights_bytes(64, 2, 8, 0) == 0
    assert L.ethos_query_proj_prepared(16, 16, None, 0, 16, 16, 16, 4, 64, 2, 8, 1, 16, 1 << 30, 16, None) == -3
    assert L.ethos_query_proj_prepared(16, 16, 16, need - 1, 16, 16, 16, 4, 64, 2, 8, 1, 16, 1 << 30, 16, None) == -5
    assert L.ethos_query_proj_prepare(16, 64, 2, 8, 1, 16, need - 1, None) == -5
    assert L.ethos_query_proj_prepare(None, 64, 2, 8, 1, 16, need, None) == -3
    assert L.ethos_query_proj_prepare(None, 64, 2, 8, 0, None, 0, None) == 0
    # workspace too small
    assert L.ethos_sort_segment(1, 100, 16, 16, 8, 16, 16, 16, 16, 16, 16, None) == -5
    # misaligned apply pointers
    assert L.ethos_apply_scatter(3, 16, 16, 16, 16, 16, 16, 16, 4, 2, 2, 64, 32, 1, 16, 1 << 30, 16, None) == -4
    # apply workspace too small
    assert L.ethos_apply_scatter(16, 16, 16, 16, 16, 16, 16, 16, 4, 2, 2, 64, 32, 1, 16, 8, 16, None) == -5
    # unsupported generator shape
    assert L.ethos_generate(16, 4, 16, 16, 4, 16, 16, 10, 32, 64, 1, 16, 16, None) == -6
    # zero-size work is a no-op success
    assert L.ethos_query_proj(None, None, None, None, None, 0, 8, 2, 8, 1, None, 0, None, None) == 0
    assert L.ethos_last_error() == b""


def test_workspace_size_grows_with_pairs():
    L = _lib.load()
    a = L.ethos_sort_workspace_bytes(1000, 262144)
    b = L.ethos_sort_workspace_bytes(1_000_000, 262144)
    assert 16 * 1000 <= a < b and b >= 16 * 1_000_000


@pytest.mark.parametrize("n", [1, 7, 4096, 4097, 524288, 4194304])
def test_workspace_helper_covers_requested_bytes(n):
    """The sort workspace handed to the ABI is at least what the library asks for."""
    import torch

    from ethos_amd import hip

    need = _lib.load().ethos_sort_workspace_bytes(n, 262144)
    ws, size = hip.workspace(need, torch.device("cpu"))
    assert size == ws.numel() * ws.element_size() >= need


def test_route_rejects_top_k_above_32():
    L = _lib.load()
    # more than 512 sub-keys and misaligned tables are rejected as well
    assert L.ethos_route_topk(16, 16, 16, None, 4, 32, 1024, 4, 8, 1, 16, 16, None) == -6
    assert L.ethos_route_topk(18, 16, 16, None, 4, 32, 64, 4, 8, 1, 16, 16, None) == -4
    assert L.ethos_route_topk(16, 16, 16, None, 4, 32, 4096, 40, 32, 1, 16, 16, None) == -6


def test_route_prepared_keys_argument_errors():
    L = _lib.load()
    n = L.ethos_route_keys_bytes(512, 256, 1)
    assert n == 2 * 512 * 128 * 2
    assert L.ethos_route_keys_bytes(200, 64, 0) == 2 * 224 * 32 * 4  # keys padded to blocks of 32
    assert L.ethos_route_keys_bytes(1024, 256, 1) == 0 and L.ethos_route_keys_bytes(512, 250, 1) == 0
    assert L.ethos_route_keys_bytes(512, 256, 7) == 0
    assert L.ethos_route_prepare_keys(16, 16, 512, 256, 7, 16, n, None) == -1
    assert L.ethos_route_prepare_keys(16, 16, 1024, 256, 1, 16, n, None) == -6
    assert L.ethos_route_prepare_keys(16, None, 512, 256, 1, 16, n, None) == -3
    assert L.ethos_route_prepare_keys(16, 16, 512, 256, 1, 16, n - 1, None) == -2
    assert L.ethos_route_prepare_keys(16, 16, 512, 256, 1, 18, n, None) == -4
    args = (16, 16, 16, None)
    assert L.ethos_route_topk_prepared(*args, None, n, 4, 256, 512, 4, 8, 1, 16, 16, None) == -3
    assert L.ethos_route_topk_prepared(*args, 16, n - 1, 4, 256, 512, 4, 8, 1, 16, 16, None) == -2
    assert L.ethos_route_topk_prepared(*args, 18, n, 4, 256, 512, 4, 8, 1, 16, 16, None) == -4
    assert L.ethos_route_topk_prepared(*args, 16, n, 4, 256, 512, 40, 32, 1, 16, 16, None) == -6
    assert L.ethos_route_topk_prepared(*args, 16, n, 0, 256, 512, 4, 8, 1, 16, 16, None) == 0  # no rows: nothing to do


def test_sort_segment_token_proj_argument_errors():
    """Checked before any HIP call, so no GPU is needed."""
    L = _lib.load()
    ok = [16, 100, 262144, 16, 1 << 20, 16, 16, 16, 16, 16, 16, 16, 16, 16, 10, 64, 32, 1, 16, None]
    bad_dtype = list(ok)
    bad_dtype[17] = 5
    assert L.ethos_sort_segment_token_proj(*bad_dtype) == -1
    bad_width = list(ok)
    bad_width[15] = 60  # d_model not a multiple of 8 (bf16)
    assert L.ethos_sort_segment_token_proj(*bad_width) == -6
    no_x = list(ok)
    no_x[11] = None
    assert L.ethos_sort_segment_token_proj(*no_x) == -3
    misaligned = list(ok)
    misaligned[18] = 18
    assert L.ethos_sort_segment_token_proj(*misaligned) == -4
    assert b"ethos_sort_segment_token_proj" in L.ethos_last_error()


def test_sort_noalloc_rejects_pairs_beyond_its_static_workspace():
    """The no-allocation sort takes at most NOALLOC_MAX_PAIRS pairs (checked before any
    HIP call, so no GPU is needed), and validates like ethos_sort_segment."""
    L = _lib.load()
    n = _lib.NOALLOC_MAX_PAIRS + 1
    assert L.ethos_sort_segment_noalloc(16, n, 262144, 16, 16, 16, 16, 16, 16, None) == -2
    assert b"static workspace" in L.ethos_last_error()
    assert L.ethos_sort_segment_noalloc(16, 100, 0, 16, 16, 16, 16, 16, 16, None) == -2
    assert L.ethos_sort_segment_noalloc(None, 100, 262144, 16, 16, 16, 16, 16, 16, None) == -3
    # the static array covers the library's own workspace formula at the limit
    assert L.ethos_sort_workspace_bytes(_lib.NOALLOC_MAX_PAIRS, 262144) <= 20 * 2 ** 20


def test_expert_forward_argument_errors():
    L = _lib.load()
    args = [16, 16, 256, 16, 16, None, None, 16, 16, 16, 64, 16, 16, 16, 16, 48, 2, 4, 16, 32, 64]
    ws = L.ethos_expert_forward_workspace_bytes(48, 2, 4, 64, 64, 32, 1, 0)
    assert ws > 48 * 32 * 2 + 64 * 64 * 2
    assert L.ethos_expert_forward_workspace_bytes(48, 2, 4, 64, 64, 32, 1, 1) != ws
    # unknown dtype, bad order, unsupported d_latent, null pointer, small workspace, misaligned
    assert L.ethos_expert_forward(*args, 7, 0, 16, ws, 16, 16, None) == -1
    assert L.ethos_expert_forward(*args, 1, 2, 16, ws, 16, 16, None) == -2
    bad = list(args)
    bad[18] = 10
    assert L.ethos_expert_forward(*bad, 1, 0, 16, ws, 16, 16, None) == -6
    assert L.ethos_expert_forward(*args, 1, 0, None, ws, 16, 16, None) == -3
    noseg = list(args)
    noseg[8] = None  # seg_off
    assert L.ethos_expert_forward(*noseg, 1, 0, 16, ws, 16, 16, None) == -3
    assert L.ethos_expert_forward(*args, 1, 0, 16, 8, 16, 16, None) == -5
    assert L.ethos_expert_forward(*args, 1, 0, 16, ws, 18, 16, None) == -4
    # an empty batch is a no-op success
    empty = list(args)
    empty[15] = 0
    assert L.ethos_expert_forward(*empty, 1, 0, None, 0, None, None, None) == 0
    # a misaligned caller-provided token projection
    misx = list(args)
    misx[6] = 18
    assert L.ethos_expert_forward(*misx, 1, 0, 16, ws, 16, 16, None) == -4


def test_expert_backward_argument_errors():
    L = _lib.load()
    ws = L.ethos_expert_backward_workspace_bytes(48, 2, 4, 64)
    assert ws >= 48 * 2 * 4 * 8  # the per-pair scalars at least
    assert L.ethos_expert_backward_workspace_bytes(-1, 2, 4, 64) == 0
    args = [16, 16, 16, 16, 16, 16, 16, 16, 48, 2, 4, 64]
    outs = [16, 16, 16, 16, None]
    assert L.ethos_expert_backward(*args, 7, 16, ws, *outs) == -1
    assert L.ethos_expert_backward(*args, 1, 16, ws - 16, *outs) == -5
    noperm = list(args)
    noperm[4] = None
    assert L.ethos_expert_backward(*noperm, 1, 16, ws, *outs) == -3
    assert L.ethos_expert_backward(*args, 1, None, ws, *outs) == -3
    assert L.ethos_expert_backward(*args, 1, 24, ws, *outs) == -4
    bad = list(args)
    bad[11] = 60
    assert L.ethos_expert_backward(*bad, 1, 16, ws, *outs) == -6
    empty = list(args)
    empty[8] = 0
    assert L.ethos_expert_backward(*empty, 1, None, 0, None, None, None, None, None) == 0


def test_token_proj_argument_errors():
    L = _lib.load()
    assert L.ethos_token_proj(16, 16, 16, 4, 64, 32, 7, 16, None) == -1
    assert L.ethos_token_proj(16, 16, 16, -1, 64, 32, 1, 16, None) == -2
    assert L.ethos_token_proj(16, 16, 16, 4, 60, 32, 1, 16, None) == -6
    assert L.ethos_token_proj(None, 16, 16, 4, 64, 32, 1, 16, None) == -3
    assert L.ethos_token_proj(16, 16, 16, 4, 64, 32, 1, 18, None) == -4
    # bf16 with d_model % 64 == 0 needs W_u^T
    assert L.ethos_token_proj(16, 16, None, 4, 64, 32, 1, 16, None) == -3
    assert L.ethos_token_proj(None, None, None, 0, 64, 32, 1, None, None) == 0


def test_stage_events_argument_errors():
    L = _lib.load()
    assert L.ethos_stage_events(None, 17) == -2
    assert L.ethos_stage_events(None, 2) == -2
    assert L.ethos_stage_events(None, 0) == 0
