"""Helpers to load the reference-generated golden fixtures (tests/golden/*.npz)."""
import hashlib
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = ["tiny", "tiny_signal", "tiny_fp32", "tiny_fp32_signal", "cfg1", "cfg1_signal", "cfg1_dq128",
            "cfg3", "cfg3_signal"]


def load(name):
    f = np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)
    meta = json.loads(str(f["meta"]))
    return f, meta


def sha_of(t):
    import torch

    t = t.detach().contiguous()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return hashlib.sha256(t.numpy().tobytes()).hexdigest()
