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


def apply_from_routing(P: dict, x: torch.Tensor, gates: torch.Tensor, ids: torch.Tensor, n_heads: int,
                       chunk: int = 2048):
    """The expert stages of model.py:312-341 in float32 for a given routing (gates and ids
    [n, H, k]), on x's device: y [n, d], and each token's scale sqrt(sum_p |a_p|^2 |v_p|^2) / H,
    the size of its terms (an error measured against it does not grow where the terms cancel).
    The hidden rows and v rows are computed once per distinct expert; the pairs in token chunks."""
    n, d = x.shape
    W1 = P["generation_network.net.0.weight"].float()
    W2 = P["generation_network.net.2.weight"].float()
    uniq, inv = torch.unique(ids.reshape(-1).long(), return_inverse=True)
    hid = F.gelu(P["expert_latents.weight"][uniq].float() @ W1.t())   # [U, dh]
    v = hid @ W2[d:].t()                                               # [U, d]
    vn = v.norm(dim=1)
    xp = x.float() @ W2[:d]                                            # [n, dh]
    inv = inv.view(ids.shape)
    y = torch.empty((n, d), dtype=torch.float32, device=x.device)
    scale = torch.empty(n, dtype=torch.float32, device=x.device)
    for t0 in range(0, n, chunk):
        sl = inv[t0:t0 + chunk]
        c = (hid[sl] * xp[t0:t0 + chunk, None, None, :]).sum(-1)
        a = F.gelu(c) * gates[t0:t0 + chunk].float()
        y[t0:t0 + chunk] = (a.unsqueeze(-1) * v[sl]).sum(dim=(1, 2)) / n_heads
        scale[t0:t0 + chunk] = torch.sqrt(((a * vn[sl]) ** 2).sum(dim=(1, 2))) / n_heads
    return y, scale


# ----------------------------------------------------------------- whole language model
def _rms(x, w, eps):
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * xf.to(x.dtype)


def _rot_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def _attention(P, pre, x, cfg):
    """DeepseekV3Attention.forward (model.py:103-165) on its matmul + additive-mask path."""
    b, n, _ = x.shape
    H, nope, rope, vd = cfg.num_heads, cfg.qk_nope_head_dim, cfg.qk_rope_head_dim, cfg.v_head_dim
    qd = nope + rope
    eps = cfg.rms_norm_eps
    q = F.linear(_rms(F.linear(x, P[pre + "q_a_proj.weight"]), P[pre + "q_a_layernorm.weight"], eps),
                 P[pre + "q_b_proj.weight"]).view(b, n, H, qd)
    q_nope, q_pe = q[..., :nope], q[..., nope:]
    ckv = F.linear(x, P[pre + "kv_a_proj_with_mqa.weight"])
    c, k_pe = ckv[..., : cfg.kv_lora_rank], ckv[..., cfg.kv_lora_rank:]
    kv = F.linear(_rms(c, P[pre + "kv_a_layernorm.weight"], eps), P[pre + "kv_b_proj.weight"]).view(b, n, H, nope + vd)
    k_nope, v = kv[..., :nope], kv[..., nope:]
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, rope, 2).float() / rope))
    f = torch.outer(torch.arange(n).float(), inv)
    emb = torch.cat((f, f), dim=-1)
    cos, sin = emb.cos().to(x.dtype), emb.sin().to(x.dtype)
    qp = q_pe.transpose(1, 2)
    kp = k_pe.view(b, n, 1, rope).transpose(1, 2)
    qp = qp * cos + _rot_half(qp) * sin
    kp = kp * cos + _rot_half(kp) * sin
    Q = torch.cat([q_nope.transpose(1, 2), qp], dim=-1)
    K = torch.cat([k_nope.transpose(1, 2), kp.expand(b, H, n, rope)], dim=-1)
    mask = torch.triu(torch.full((n, n), float("-inf")), diagonal=1)
    w = torch.matmul(Q, K.transpose(-2, -1)) * qd ** (-0.5) + mask
    w = F.softmax(w, dim=-1, dtype=torch.float32).to(Q.dtype)
    o = torch.matmul(w, v.transpose(1, 2)).transpose(1, 2).reshape(b, n, H * vd)
    return F.linear(o, P[pre + "o_proj.weight"])


def lm_forward(P: dict, ids: torch.Tensor, cfg, routing: dict):
    """CompressedMoEModel.forward (model.py:384-396) in float32; the expert layer of block i
    uses the imposed expert ids routing[i] ([n_tok, H, k])."""
    eps = cfg.rms_norm_eps
    h = P["tok_embeddings.weight"][ids]
    b, n, d = h.shape
    for i in range(cfg.num_layers):
        pre = f"layers.{i}."
        hh = h + _attention(P, pre + "self_attn.", _rms(h, P[pre + "input_layernorm.weight"], eps), cfg)
        z = _rms(hh, P[pre + "post_attention_layernorm.weight"], eps)
        if i < cfg.num_dense_layers:
            mp = pre + "mlp."
            m = F.linear(F.silu(F.linear(z, P[mp + "w1.weight"])) * F.linear(z, P[mp + "w3.weight"]),
                         P[mp + "w2.weight"])
        else:
            sub = {k[len(pre + "mlp."):]: v for k, v in P.items() if k.startswith(pre + "mlp.")}
            y, _ = layer_forward(sub, z.reshape(-1, d), cfg.num_routing_heads, cfg.top_k, bn_batch_stats=False,
                                 ids=routing[i])
            m = y.view(b, n, d)
        h = hh + m
    return F.linear(_rms(h, P["norm.weight"], eps), P["output.weight"])
