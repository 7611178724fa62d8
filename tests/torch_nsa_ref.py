"""Differentiable float64 torch formulation of the NSAAttention forward, used by the
GPU tests to check the module's gradients with torch autograd.

It follows the reference module (nsa/kernels.py:2119-2208 compress_tokens with the
per-block MLP, :2210-2478 forward) but evaluates each branch as dense masked
softmax attention; the selection indices are an input (the top-n is not
differentiable).  Test infrastructure only.
"""
import math

import torch


def dense_branch(q, k, v, mask, scale):
    """q [B,H,T,dk], k [B,G,Tk,dk], v [B,G,Tk,dv], mask [B,H,T,Tk] bool."""
    H, G = q.shape[1], k.shape[1]
    ke = k.repeat_interleave(H // G, 1)
    ve = v.repeat_interleave(H // G, 1)
    s = (q @ ke.transpose(-1, -2)) * scale
    s = s.masked_fill(~mask, float("-inf"))
    p = torch.softmax(s, -1).nan_to_num(0.0)
    return p @ ve


def nsa_forward(x, P, cfg, indices):
    """x [B,T,D] float64 (requires_grad as needed); P: dict name -> float64 tensor;
    indices [B,G,T,n] int64.  Returns [B,T,D]."""
    B, T, D = x.shape
    H, G, dk, dv = cfg.n_heads, cfg.n_kv_groups, cfg.head_dim_qk, cfg.head_dim_v
    lin = torch.nn.functional.linear

    def proj(name, n, w):
        return lin(x, P[name + ".weight"], P.get(name + ".bias")).view(B, T, n, w).transpose(1, 2)

    q = proj("q_proj", H, dk)
    kc_in, vc_in = proj("k_compress", G, dk), proj("v_compress", G, dv)
    ks, vs = proj("k_select", G, dk), proj("v_select", G, dv)
    kw, vw = proj("k_sliding", G, dk), proj("v_sliding", G, dv)
    scale = 1.0 / math.sqrt(dk)
    # compress_tokens
    n_act = (T - cfg.l) // cfg.d + 1
    kcs, vcs, be = [], [], []
    pos = P["pos_embed.weight"]
    for i in range(max(n_act, 0)):
        st = i * cfg.d
        blk = kc_in[:, :, st:st + cfg.l]
        xin = torch.cat([blk, pos[:cfg.l].view(1, 1, cfg.l, cfg.l).expand(B, G, cfg.l, cfg.l)], -1)
        h = torch.relu(lin(xin, P["compress_mlp.0.weight"], P.get("compress_mlp.0.bias")))
        kcs.append(lin(h, P["compress_mlp.2.weight"], P.get("compress_mlp.2.bias")).mean(2))
        vcs.append(vc_in[:, :, st:st + cfg.l].mean(2))
        be.append(i * cfg.d + cfg.l - 1)
    t = torch.arange(T)
    outs = []
    if n_act > 0:
        kc = torch.stack(kcs, 2)
        vc = torch.stack(vcs, 2)
        m = (torch.tensor(be).view(1, -1) <= t.view(-1, 1)).expand(B, H, T, n_act)
        outs.append(dense_branch(q, kc, vc, m, scale))
    else:
        outs.append(torch.zeros(B, H, T, dv, dtype=x.dtype))
    # selection with the wrapper's all-invalid fallback
    idx = indices.clone()
    allneg = (idx < 0).all(-1)
    idx[allneg] = (t.view(1, 1, T).expand_as(allneg)[allneg] // cfg.l_prime).unsqueeze(-1).expand(-1, idx.shape[-1])
    blk_of = t // cfg.l_prime
    nb = int(blk_of.max()) + 1
    sel = torch.zeros(B, G, T, nb + 1, dtype=torch.bool)
    sel.scatter_(-1, torch.where(idx < 0, torch.full_like(idx, nb), idx.clamp(max=nb)), True)
    m = sel[..., blk_of] & (t.view(1, -1) <= t.view(-1, 1))
    outs.append(dense_branch(q, ks, vs, m.repeat_interleave(H // G, 1), scale))
    mw = (t.view(1, -1) <= t.view(-1, 1)) & (t.view(1, -1) > t.view(-1, 1) - cfg.w)
    outs.append(dense_branch(q, kw, vw, mw.expand(B, H, T, T), scale))
    gl = lin(torch.relu(lin(x, P["gate_mlp.0.weight"], P.get("gate_mlp.0.bias"))), P["gate_mlp.2.weight"],
             P.get("gate_mlp.2.bias")).view(B, T, H, 3).permute(0, 2, 1, 3)
    gates = torch.softmax(gl, -1) if cfg.gate_mode == "softmax" else torch.sigmoid(gl)
    o = outs[0] * gates[..., 0:1] + outs[1] * gates[..., 1:2] + outs[2] * gates[..., 2:3]
    o = o.transpose(1, 2).reshape(B, T, H * dv)
    return lin(o, P["o_proj.weight"], P.get("o_proj.bias"))
