"""Loop-faithful CPU restatement of the reference expert layer -- for tests and the CPU baseline only.

Times what the reference's own CPU path costs (bench.py's ``cpu_baseline`` leg) and
never runs in the product.  It performs the reference's operations in the
reference's order and dtype, written here from the algorithm:

  router (model.py:214-252), per head: Linear + bias, BatchNorm (eval), split in
    halves, scores against both sub-key tables, top-2k per half, 2k x 2k dtype sums,
    top-k, fp32 softmax cast to dtype, decode e = i1 * K + i2;
  layer (model.py:303-341): for head, for token, for each of its k experts --
    hidden = gelu(latent @ W1^T-part), token projection x @ W_u, scalar
    gelu(hidden . projection) * gate, contribution scalar * (hidden @ W_v) added to
    an fp32 accumulator; the accumulator is cast per head, heads summed in dtype,
    and the sum divided by the head count.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def route(x: torch.Tensor, sd: dict, n_heads: int, top_k: int):
    K = sd["router.sub_keys_1.weight"].shape[0]
    keys_a = sd["router.sub_keys_1.weight"]
    keys_b = sd["router.sub_keys_2.weight"]
    cand = 2 * top_k
    gates, experts = [], []
    for h in range(n_heads):
        pre = "router.query_norms.%d." % h
        q = F.linear(x, sd["router.query_projs.%d.weight" % h], sd["router.query_projs.%d.bias" % h])
        q = F.batch_norm(q, sd[pre + "running_mean"], sd[pre + "running_var"], sd[pre + "weight"], sd[pre + "bias"],
                         False, 0.0, 1e-5)
        half = q.shape[-1] // 2
        va, ia = torch.topk(q[:, :half] @ keys_a.t(), cand, dim=-1)
        vb, ib = torch.topk(q[:, half:] @ keys_b.t(), cand, dim=-1)
        grid = (va[:, :, None] + vb[:, None, :]).reshape(x.shape[0], cand * cand)
        best, where = torch.topk(grid, top_k, dim=-1)
        gates.append(F.softmax(best, dim=-1, dtype=torch.float32).to(x.dtype))
        experts.append(ia.gather(1, where // cand) * K + ib.gather(1, where % cand))
    return torch.stack(gates, 1), torch.stack(experts, 1)


def layer(x: torch.Tensor, sd: dict, n_heads: int, top_k: int) -> torch.Tensor:
    """x [n, d] -> y [n, d], one (head, token, k) iteration at a time."""
    n, d = x.shape
    gates, experts = route(x, sd, n_heads, top_k)
    latents = sd["expert_latents.weight"]
    w1t = sd["generation_network.net.0.weight"].t()
    w2t = sd["generation_network.net.2.weight"].t()
    w_u = w2t[:, :d].t()
    w_v = w2t[:, d:]
    total = torch.zeros_like(x)
    for h in range(n_heads):
        per_head = torch.zeros_like(x)
        for t in range(n):
            xt = x[t]
            acc = torch.zeros(d)
            for j in range(top_k):
                hid = F.gelu(latents[experts[t, h, j]] @ w1t)
                act = F.gelu(torch.dot(hid, xt @ w_u)) * gates[t, h, j]
                acc += act * (hid @ w_v)
            per_head[t] = acc
        total += per_head
    return total / n_heads
