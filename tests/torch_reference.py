"""A vectorised float32 PyTorch restatement of the reference's router and layer
(model.py:208-254 ProductKeyRouter.forward, model.py:288-343 SimplifiedHypernetMoE.forward),
used to check gradients: autograd through it gives the reference's gradients.

The loops of model.py:312-341 are sums, written here as tensor reductions; the routing
selection can be imposed (`ids`), in which case the selected scores are gathered from the
same sub-scores the reference's topk values come from (model.py:220-234)."""
import torch
import torch.nn.functional as F


def leaves(sd: dict) -> dict:
    """float32 copies of a state_dict; floating parameters require grad, buffers do not."""
    out = {}
    for k, v in sd.items():
        t = v.detach().clone()
        if t.is_floating_point():
            t = t.float()
            if not (k.endswith("running_mean") or k.endswith("running_var")):
                t.requires_grad_(True)
        out[k] = t
    return out


def layer_forward(P: dict, x: torch.Tensor, n_heads: int, top_k: int, bn_batch_stats: bool, ids=None,
                  eps: float = 1e-5):
    """y [n, d] of the reference layer for x [n, d] (float32), and the expert ids [n, H, k]."""
    n, d = x.shape
    K1 = P["router.sub_keys_1.weight"]
    K2 = P["router.sub_keys_2.weight"]
    K = K1.shape[0]
    k_cand = 2 * top_k
    gates, experts = [], []
    for h in range(n_heads):
        q = F.linear(x, P[f"router.query_projs.{h}.weight"], P[f"router.query_projs.{h}.bias"])
        pre = f"router.query_norms.{h}."
        q = F.batch_norm(q, None if bn_batch_stats else P[pre + "running_mean"],
                         None if bn_batch_stats else P[pre + "running_var"], P[pre + "weight"], P[pre + "bias"],
                         bn_batch_stats, 0.0, eps)
        q1, q2 = q.chunk(2, dim=-1)
        s1 = q1 @ K1.t()
        s2 = q2 @ K2.t()
        if ids is None:
            t1, i1 = torch.topk(s1, k_cand, dim=-1)
            t2, i2 = torch.topk(s2, k_cand, dim=-1)
            comb = (t1.unsqueeze(2) + t2.unsqueeze(1)).view(n, -1)
            fs, ci = torch.topk(comb, top_k, dim=-1)
            e = i1.gather(1, ci // k_cand) * K + i2.gather(1, ci % k_cand)
        else:
            e = ids[:, h].long()
            fs = s1.gather(1, e // K) + s2.gather(1, e % K)
        gates.append(F.softmax(fs, dim=-1, dtype=torch.float32))
        experts.append(e)
    g = torch.stack(gates, dim=1)           # [n, H, k]
    e = torch.stack(experts, dim=1)
    W1 = P["generation_network.net.0.weight"]   # [dh, dl]
    W2 = P["generation_network.net.2.weight"]   # [2d, dh]
    z = P["expert_latents.weight"][e]           # [n, H, k, dl]
    hid = F.gelu(z @ W1.t())                    # h_i = gelu(z_i W1)
    xp = x @ W2[:d]                             # x_proj = x W_u, W_u = W2[:d]  [d, dh]
    c = (hid * xp[:, None, None, :]).sum(-1)
    a = F.gelu(c) * g
    v = hid @ W2[d:].t()                        # h_i W_v, W_v = W2[d:]^T
    y = (a.unsqueeze(-1) * v).sum(dim=2).sum(dim=1) / n_heads
    return y, e
