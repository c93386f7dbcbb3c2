"""The language model (ethos_amd.model.CompressedMoEModel) on the GPU:

  - the small model (one dense block, two expert blocks) against the reference's own
    logits (tests/golden/lm_tiny.npz, CompressedMoEModel in eval mode, model.py:367-396)
    in float32 and bfloat16, and against the float32 restatement of the reference model
    (tests/torch_reference.lm_forward, pinned to those logits) with the GPU run's routing
    imposed;
  - the whole-model workload at its own size (12 expert blocks, d_model 1024, MLA 16 heads,
    vocab 100,277, 4 x 2048 tokens, bf16): finite, run-to-run identical logits, and in
    every block the expert layer's queries, routing (every row: ids and gates) and output
    (a token subset) against the oracle, on the inputs that block received."""
import json
import os

import numpy as np
import pytest
import torch

from ethos_amd.layer import EthosExpertLayer
from ethos_amd.model import CompressedMoEModel, init_random_, lm_config
from ethos_amd.workloads import make_lm_inputs
from golden_util import GOLDEN
from gpu_util import check_all_tokens, check_out, to_host
from oracle import oracle as O
from torch_reference import lm_forward

pytestmark = pytest.mark.gpu


def _nerr(a, b):
    a = torch.as_tensor(np.asarray(a.detach().float().cpu() if torch.is_tensor(a) else a), dtype=torch.float64)
    b = torch.as_tensor(np.asarray(b.detach().float().cpu() if torch.is_tensor(b) else b), dtype=torch.float64)
    return float((a - b).norm() / b.norm())


def _fixture():
    f = np.load(os.path.join(GOLDEN, "lm_tiny.npz"), allow_pickle=False)
    return f, json.loads(str(f["meta"]))


def _bf16(a):
    return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).float()


def _run(m, ids):
    """Logits and the input each expert block received."""
    inputs = {}
    hooks = [blk.mlp.register_forward_pre_hook(lambda mod, a, i=i: inputs.__setitem__(i, a[0].detach()))
             for i, blk in enumerate(m.layers) if isinstance(blk.mlp, EthosExpertLayer)]
    try:
        with torch.no_grad():
            logits = m(ids.cuda())
    finally:
        for h in hooks:
            h.remove()
    return logits, inputs


def _small(dtype):
    f, meta = _fixture()
    cfg, sd, ids = make_lm_inputs(seed=meta["seed"], batch=meta["batch"], seq=meta["seq"])
    m = CompressedMoEModel(cfg)
    m.load_state_dict(sd)
    return f, cfg, sd, ids, m.to(dtype).cuda().eval()


def test_lm_matches_reference_logits_fp32():
    f, cfg, sd, ids, m = _small(torch.float32)
    logits, inputs = _run(m, ids)
    assert logits.shape == (2, 24, cfg.vocab_size) and logits.dtype == torch.float32
    e = _nerr(logits, f["ref_logits_fp32"])
    # each expert block's routing of the input it received, against the reference's choice
    agree = {}
    for i, x in inputs.items():
        ids_i = m.layers[i].mlp.router(x.reshape(-1, cfg.d_model))[1].cpu().numpy()
        agree[i] = int(np.all(ids_i == f[f"ref_ids_fp32_{i}"], axis=-1).sum())
    print(f"lm fp32: logits normalised error {e:.2e} vs the reference; routing rows equal per block {agree} "
          f"of {ids.numel() * cfg.num_routing_heads}")
    assert e < 1e-4, e
    assert all(v == ids.numel() * cfg.num_routing_heads for v in agree.values())


def test_lm_bf16_close_to_reference_logits():
    f, cfg, sd, ids, m = _small(torch.bfloat16)
    logits, _ = _run(m, ids)
    assert logits.dtype == torch.bfloat16
    e16 = _nerr(logits, _bf16(f["ref_logits_bf16"]))
    e32 = _nerr(logits, f["ref_logits_fp32"])
    e_ref = _nerr(_bf16(f["ref_logits_bf16"]), f["ref_logits_fp32"])
    print(f"lm bf16: normalised error {e32:.2e} vs the reference's fp32 logits (the reference's own bf16 run: "
          f"{e_ref:.2e}), {e16:.2e} vs the reference's bf16 logits")
    # at least as close to the float32 logits as the reference's own bf16 run, and the two
    # bf16 runs (different rounding sequences of the same model) within twice that
    assert e32 < 3e-2 and e32 <= e_ref
    assert e16 <= 2 * e_ref


def test_lm_matches_restatement_with_imposed_routing_fp32():
    f, cfg, sd, ids, m = _small(torch.float32)
    logits, inputs = _run(m, ids)
    with torch.no_grad():
        routing = {i: m.layers[i].mlp.router(x.reshape(-1, cfg.d_model))[1].cpu() for i, x in inputs.items()}
        ref = lm_forward({k: v.float() for k, v in sd.items()}, ids, cfg, routing)
    assert _nerr(logits, ref) < 1e-4


def test_lm_whole_model_workload_full_size():
    """12 expert blocks, d_model 1024, 4 x 2048 tokens, bf16, random init (seed 0)."""
    cfg = lm_config()
    m = init_random_(CompressedMoEModel(cfg), seed=0).to(torch.bfloat16).cuda().eval()
    ids = torch.randint(0, cfg.vocab_size, (4, 2048), generator=torch.Generator().manual_seed(0))
    logits, inputs = _run(m, ids)
    logits2, _ = _run(m, ids)
    torch.cuda.synchronize()
    assert logits.shape == (4, 2048, cfg.vocab_size)
    assert bool(torch.isfinite(logits).all())
    assert torch.equal(logits.view(torch.int16), logits2.view(torch.int16)), "logits differ between two runs"
    del logits2
    assert len(inputs) == cfg.num_layers
    n = ids.numel()
    q_sub = np.arange(0, n, 4)     # 2,048 tokens for the query projection
    y_sub = np.arange(7, n, 64)    # 128 tokens for the layer output
    for i, x in sorted(inputs.items()):
        layer = m.layers[i].mlp
        xf = x.reshape(-1, cfg.d_model).contiguous()
        with torch.no_grad():
            q = layer.router.queries(xf)
            gates, ids_l = layer.router.route(xf)
            y = layer.forward_flat(xf)
        torch.cuda.synchronize()
        P = O.unpack_state({k: v.cpu() for k, v in layer.state_dict().items()}, cfg.num_routing_heads)
        xs, qh = to_host(xf), to_host(q)
        assert np.array_equal(qh[q_sub], O.query_proj(xs[q_sub], P["Wq"], P["bq"], P["alpha"], P["beta"], "bf16"))
        g_ref, ids_ref = O.route(qh, P["K1"], P["K2"], cfg.top_k, "bf16")
        ih, gh = to_host(ids_l), to_host(gates)
        rows = int(np.any(ih != ids_ref, -1).sum())
        print(f"block {i}: {rows} of {ih.shape[0] * ih.shape[1]} routing rows differ from the oracle, "
              f"{int(np.count_nonzero(gh != g_ref))} gates", flush=True)
        assert rows == 0 and np.array_equal(gh, g_ref)
        r = O.layer_forward(xs, P, cfg.num_routing_heads, cfg.top_k, "bf16", tokens=y_sub, q=qh,
                            routed=(g_ref, ids_ref))
        check_out(O.to_f32(to_host(y), "bf16")[y_sub], r["out"], "bf16", nerr_max=2e-3)
        check_all_tokens(layer, xf, gates, ids_l, y, f"block {i}")
