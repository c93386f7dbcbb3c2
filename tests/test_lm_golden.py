"""The whole-model fixture (tests/golden/lm_tiny.npz, the reference's CompressedMoEModel,
model.py:367-396, in eval mode on its matmul attention path): it still matches the
regenerated inputs, and the float32 test-side restatement of the model
(tests/torch_reference.lm_forward), fed the reference's own expert routing, reproduces the
reference's logits.  CPU only."""
import json
import os

import numpy as np
import torch

from ethos_amd.workloads import make_lm_inputs
from golden_util import GOLDEN, sha_of
from torch_reference import lm_forward


def _load():
    f = np.load(os.path.join(GOLDEN, "lm_tiny.npz"), allow_pickle=False)
    return f, json.loads(str(f["meta"]))


def _nerr(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def test_lm_inputs_regenerate_identically():
    f, meta = _load()
    cfg, sd, ids = make_lm_inputs(seed=meta["seed"], batch=meta["batch"], seq=meta["seq"])
    assert np.array_equal(ids.numpy(), f["in_ids"])
    for k, v in sd.items():
        assert str(f["sha_" + k]) == sha_of(v), k


def test_lm_restatement_reproduces_reference_logits():
    f, meta = _load()
    cfg, sd, ids = make_lm_inputs(seed=meta["seed"], batch=meta["batch"], seq=meta["seq"])
    P = {k: v.float() for k, v in sd.items()}
    routing = {i: torch.from_numpy(f[f"ref_ids_fp32_{i}"]) for i in range(cfg.num_dense_layers, cfg.num_layers)}
    with torch.no_grad():
        logits = lm_forward(P, ids, cfg, routing)
    ref = f["ref_logits_fp32"]
    assert logits.shape == ref.shape
    e = _nerr(logits.numpy(), ref)
    assert e < 1e-5, e
    # the expert layers show in the logits: without their v half the logits move by > 1e-2
    P0 = dict(P)
    for i in routing:
        k = f"layers.{i}.mlp.generation_network.net.2.weight"
        w = P0[k].clone()
        w[cfg.d_model:] = 0
        P0[k] = w
    with torch.no_grad():
        assert _nerr(lm_forward(P0, ids, cfg, routing).numpy(), ref) > 1e-2
