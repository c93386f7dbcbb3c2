"""Write golden fixtures from the reference's own PyTorch expert layer.

Run in the build container only (the reference tree is not present on GPU machines):

    python tests/golden/make_golden.py        # the expert-layer fixtures
    python tests/golden/make_golden.py lm     # the whole-model fixture (lm_tiny.npz)

The reference (wrmedford/ETHOS, model.py) is imported read-only from
/root/reference, its modules are built from this repository's seeded synthetic
state dicts (ethos_amd/workloads.py), put in eval mode, and run on CPU.  For each
shape the fixture holds:

  meta          JSON: shape, seed, signal flag, torch version, thread count
  sha_*         sha256 of the regenerated inputs (tests check they still match)
  ref_scores    router gates  [n_tok, H, k]      (model.py:234,251)
  ref_indices   router experts [n_tok, H, k]     (model.py:245,252), int32
  ref_out       layer output  [n_tok, d_model]   (model.py:288-343)
  ref_q         per-head query after BatchNorm [n_tok, H, dq] (model.py:215-216), small
                shapes and the 64-token layer
  ref_s1/ref_s2 per-head sub-key scores [n_tok, H, K] (model.py:220-221), small shapes
  in_*          the inputs themselves, for the tiny shapes

Why the reference is run at all: the conventions of the path -- which query half
meets sub_keys_1, the expert id decode, which half of the generator output is
u and which v, exact-erf GELU, the fp32 per-head accumulation and the 1/H head
average -- are not fixed by any closed form, and the reference ships no tests or
vectors.  Everything the mathematics does fix is pinned by tests/ instead.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
import time

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
REF = "/root/reference"

sys.path.insert(0, REPO)
from ethos_amd.workloads import SHAPES, make_inputs  # noqa: E402

# (fixture name, shape name, signal, internals to store: "qs" = ref_q and ref_s1/ref_s2,
# "q" = ref_q only, "" = none, store inputs)
PLAN = [
    ("tiny", "tiny", False, "qs", True),
    ("tiny_signal", "tiny", True, "qs", True),
    ("tiny_fp32", "tiny_fp32", False, "qs", True),
    ("tiny_fp32_signal", "tiny_fp32", True, "qs", True),
    ("cfg1", "cfg1", False, "qs", False),
    ("cfg1_signal", "cfg1", True, "", False),
    ("cfg1_dq128", "cfg1_dq128", False, "qs", False),
    ("cfg3", "cfg3", False, "q", False),
    ("cfg3_signal", "cfg3", True, "q", False),
]


def tensor_bytes(t: torch.Tensor) -> bytes:
    t = t.detach().contiguous()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return t.numpy().tobytes()


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(tensor_bytes(t)).hexdigest()


def to_np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    if t.dtype == torch.int64:
        return t.numpy().astype(np.int32)
    return t.numpy().copy()


def main(only=None):
    sys.dont_write_bytecode = True  # the reference tree is read-only
    sys.path.insert(0, REF)
    import model as ref_model  # noqa: E402  (reference, read-only)

    for name, shape_name, signal, store_internals, store_inputs in PLAN:
        if only and name not in only:
            continue
        sh = SHAPES[shape_name]
        x, sd = make_inputs(sh, seed=0, signal=signal)
        dt = sh.torch_dtype
        layer = ref_model.SimplifiedHypernetMoE(sh.config()).to(dt)
        layer.load_state_dict(sd)
        layer.eval()
        t0 = time.time()
        with torch.no_grad():
            scores, indices = layer.router(x)
            out = layer(x.view(sh.batch, sh.n_tok // sh.batch, sh.d_model)).reshape(sh.n_tok, sh.d_model)
            qs, s1s, s2s = [], [], []
            if store_internals:
                r = layer.router
                for h in range(sh.num_heads):
                    q = r.query_norms[h](r.query_projs[h](x))
                    q1, q2 = q.chunk(2, dim=-1)
                    qs.append(q)
                    s1s.append(q1 @ r.sub_keys_1.weight.t())
                    s2s.append(q2 @ r.sub_keys_2.weight.t())
        dt_s = time.time() - t0
        rec = {
            "ref_scores": to_np(scores),
            "ref_indices": to_np(indices),
            "ref_out": to_np(out),
            "sha_x": np.array(sha(x)),
        }
        for k, v in sd.items():
            rec["sha_" + k] = np.array(sha(v))
        if store_internals:
            rec["ref_q"] = to_np(torch.stack(qs, dim=1))
        if store_internals == "qs":
            rec["ref_s1"] = to_np(torch.stack(s1s, dim=1))
            rec["ref_s2"] = to_np(torch.stack(s2s, dim=1))
        if store_inputs:
            rec["in_x"] = to_np(x)
            for k, v in sd.items():
                rec["in_" + k] = to_np(v)
        meta = dict(shape=shape_name, seed=0, signal=signal, torch=torch.__version__,
                    threads=torch.get_num_threads(), ref_seconds=round(dt_s, 3))
        rec["meta"] = np.array(json.dumps(meta))
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **rec)
        print(f"{name}: {os.path.getsize(path) / 1024:.0f} KiB, reference forward {dt_s:.2f}s", flush=True)


def lm_main():
    """The reference's whole model (CompressedMoEModel, model.py:367-396) on the small
    language model of ethos_amd.workloads (LM_TINY: one dense block, two expert blocks),
    in eval mode on its matmul + additive-mask attention path (model.py:156-163), in
    float32 and bfloat16.  lm_tiny.npz holds:

      meta                JSON: seed, batch, seq, torch version, thread count
      sha_*               sha256 of the regenerated float32 parameters
      in_ids              token ids [batch, seq]
      ref_logits_fp32     logits [batch, seq, vocab] float32
      ref_logits_bf16     logits [batch, seq, vocab] bfloat16 (model cast with .to(bf16))
      ref_ids_fp32_<i>    expert ids [batch * seq, H, k] chosen by block i's router (fp32 run)
      ref_scores_fp32_<i> its gates
    """
    from types import SimpleNamespace

    sys.dont_write_bytecode = True
    sys.path.insert(0, REF)
    import model as ref_model  # noqa: E402  (reference, read-only)

    from ethos_amd.workloads import make_lm_inputs  # noqa: E402

    seed, batch, seq = 0, 2, 24
    cfg, sd, ids = make_lm_inputs(seed=seed, batch=batch, seq=seq)
    rcfg = SimpleNamespace(**vars(cfg), use_triton=False)
    rec = {"in_ids": ids.numpy().astype(np.int32)}
    for k, v in sd.items():
        rec["sha_" + k] = np.array(sha(v))
    for dt, tag in ((torch.float32, "fp32"), (torch.bfloat16, "bf16")):
        m = ref_model.CompressedMoEModel(rcfg)
        m.load_state_dict(sd, strict=True)
        m = m.to(dt).eval()
        routed = {}
        hooks = [blk.mlp.router.register_forward_hook(
            lambda mod, inp, out, i=i: routed.__setitem__(i, out))
            for i, blk in enumerate(m.layers) if i >= cfg.num_dense_layers]
        t0 = time.time()
        with torch.no_grad():
            logits = m(ids)
        for h in hooks:
            h.remove()
        rec[f"ref_logits_{tag}"] = to_np(logits)
        if tag == "fp32":
            for i, (scores, indices) in routed.items():
                rec[f"ref_ids_fp32_{i}"] = to_np(indices)
                rec[f"ref_scores_fp32_{i}"] = to_np(scores)
        print(f"lm_tiny {tag}: reference forward {time.time() - t0:.2f}s", flush=True)
    meta = dict(seed=seed, batch=batch, seq=seq, torch=torch.__version__, threads=torch.get_num_threads())
    rec["meta"] = np.array(json.dumps(meta))
    path = os.path.join(HERE, "lm_tiny.npz")
    np.savez_compressed(path, **rec)
    print(f"lm_tiny: {os.path.getsize(path) / 1024:.0f} KiB", flush=True)


if __name__ == "__main__":
    args = sys.argv[1:]
    if args == ["lm"]:
        lm_main()
    else:
        main(args or None)
