"""CPU oracle for the NSA hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker of the HIP path.  The product (the `nsa` package and
libnsa_hip.so) never imports or calls it.

Contents
  attn_fwd / attn_bwd     per-row restatement of the three branches in float64
                          (C, nsa_oracle.c; reference nsa/reference.py:13-147, :205-254)
  score_topn              Eq. 8 -> 9 -> 10 -> top-n in fp32 with a fixed operation order
                          (C; reference nsa/kernels.py:1920-2040, :2316-2343)
  exp32                   the exp() of that pipeline
  compress_tokens         MLP pooling of K, mean pooling of V, block_ends
                          (numpy float64; reference nsa/kernels.py:2119-2208)
  derive_selection / select_topk
                          Eq. 9 and Eq. 10/top-n on given score arrays (numpy;
                          reference nsa/kernels.py:1920-2040)
  nsa_forward             the NSAAttention forward (gates, mix, o_proj) in float64,
                          with indices from score_topn (reference nsa/kernels.py:2210-2478)
"""
from __future__ import annotations

import ctypes
import math
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

SLIDING, COMPRESSION, SELECTION = 0, 1, 2

_lib = None


def build() -> Path:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def _load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        P, I, D, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_double, ctypes.c_float
        lib.oracle_attn_fwd.argtypes = [I, I, I, I, I, I, I, I, P, P, P, D, I, P, P, I, I, I, P, P, P, P]
        lib.oracle_attn_fwd.restype = I
        lib.oracle_attn_bwd.argtypes = [I, I, I, I, I, I, I, I, P, P, P, P, D, I, P, P, I, I, I, P, P, P, P]
        lib.oracle_attn_bwd.restype = I
        lib.oracle_score_topn.argtypes = [I, I, I, I, I, I, P, P, P, F, I, I, I, I, I, I, P, P, P, P]
        lib.oracle_score_topn.restype = I
        lib.oracle_exp32.argtypes = [F]
        lib.oracle_exp32.restype = F
        _lib = lib
    return _lib


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else ctypes.c_void_p(0)


def _f64(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float64))


def attn_fwd(kind, q, k, v, scale, *, window=0, block_ends=None, indices=None, lprime=64, causal=True,
             positions=None):
    """q [B,H,Tq,dk], k [B,G,Tkv,dk], v [B,G,Tkv,dv] -> (out, L, M) in float64.
    k is the (b, g, time, dk) view (i.e. the transpose of the reference's [B,G,dk,T]).
    positions (optional, [Tq] ints): the query position of each row of q (and of
    indices), to evaluate a sample of rows of a long sequence."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    B, H, Tq, dk = q.shape
    G, Tkv, dv = k.shape[1], k.shape[2], v.shape[-1]
    be = np.ascontiguousarray(block_ends, dtype=np.int32) if block_ends is not None else None
    idx = np.ascontiguousarray(indices, dtype=np.int64) if indices is not None else None
    n = idx.shape[-1] if idx is not None else 0
    out = np.zeros((B, H, Tq, dv))
    L = np.zeros((B, H, Tq))
    M = np.zeros((B, H, Tq))
    tm = np.ascontiguousarray(positions, dtype=np.int32) if positions is not None else None
    rc = _load().oracle_attn_fwd(kind, B, H, G, Tq, Tkv, dk, dv, _p(q), _p(k), _p(v), float(scale), int(window),
                                 _p(be), _p(idx), n, int(lprime), int(bool(causal)), _p(tm), _p(out), _p(L), _p(M))
    assert rc == 0
    return out, L, M


def attn_bwd(kind, q, k, v, do, scale, *, window=0, block_ends=None, indices=None, lprime=64, causal=True,
             positions=None):
    """Gradients (dq [B,H,Tq,dk], dk [B,G,Tkv,dk], dv [B,G,Tkv,dv]) in float64.
    With `positions`, rows of q / do are those query positions and dk / dv hold the
    contribution of those rows only."""
    q, k, v, do = _f64(q), _f64(k), _f64(v), _f64(do)
    B, H, Tq, dk = q.shape
    G, Tkv, dv = k.shape[1], k.shape[2], v.shape[-1]
    be = np.ascontiguousarray(block_ends, dtype=np.int32) if block_ends is not None else None
    idx = np.ascontiguousarray(indices, dtype=np.int64) if indices is not None else None
    n = idx.shape[-1] if idx is not None else 0
    dq = np.zeros_like(q)
    dkk = np.zeros_like(k)
    dvv = np.zeros_like(v)
    tm = np.ascontiguousarray(positions, dtype=np.int32) if positions is not None else None
    rc = _load().oracle_attn_bwd(kind, B, H, G, Tq, Tkv, dk, dv, _p(q), _p(k), _p(v), _p(do), float(scale),
                                 int(window), _p(be), _p(idx), n, int(lprime), int(bool(causal)), _p(tm), _p(dq),
                                 _p(dkk), _p(dvv))
    assert rc == 0
    return dq, dkk, dvv


def exp32(x):
    lib = _load()
    x = np.asarray(x, dtype=np.float32)
    return np.array([lib.oracle_exp32(float(v)) for v in x.ravel()], dtype=np.float32).reshape(x.shape)


def score_topn(q, kc, block_ends, scale, *, l=32, d=16, lprime=64, n=16, include_fixed=True, n_fixed=3,
               want_scores=False, positions=None):
    """q [B,H,T,dk], kc [B,G,dk,NB] (the reference's compressed-key layout), block_ends [NB].
    Returns indices [B,G,T,n] int64 (and p_cmp [B,H,T,NB], p_slc [B,H,T,nsel] when asked)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    kc = np.ascontiguousarray(kc, dtype=np.float32)
    be = np.ascontiguousarray(block_ends, dtype=np.int32)
    B, H, T, dk = q.shape
    G, NB = kc.shape[1], kc.shape[-1]
    s = lprime // d
    nsel = (NB + s - 1) // s
    out = np.zeros((B, G, T, n), dtype=np.int64)
    pc = np.zeros((B, H, T, NB), dtype=np.float32) if want_scores else None
    psl = np.zeros((B, H, T, nsel), dtype=np.float32) if want_scores else None
    tm = np.ascontiguousarray(positions, dtype=np.int32) if positions is not None else None
    rc = _load().oracle_score_topn(B, H, G, T, dk, NB, _p(q), _p(kc), _p(be), np.float32(scale), l, d, lprime, n,
                                   int(bool(include_fixed)), int(n_fixed), _p(tm), _p(out), _p(pc), _p(psl))
    assert rc == 0
    return (out, pc, psl) if want_scores else out


# ------------------------------------------------------------------ numpy parts
def derive_selection(p_cmp, l=32, d=16, lprime=64):
    """Eq. 9 on a score array [..., NB] (reference nsa/kernels.py:1937-1962): for each
    selection block j, the compressed scores s*j+m+n (m < l'/d, n < l/d) summed in
    (m, n) order."""
    p_cmp = np.asarray(p_cmp)
    NB = p_cmp.shape[-1]
    a, s = l // d, lprime // d
    nsel = (NB + s - 1) // s
    out = np.zeros(p_cmp.shape[:-1] + (nsel,), dtype=p_cmp.dtype)
    for j in range(nsel):
        for m in range(s):
            for nn in range(a):
                ci = s * j + m + nn
                if ci < NB:
                    out[..., j] += p_cmp[..., ci]
    return out


def select_topk(sel_scores, G, n, lprime, include_fixed=True, n_fixed=3):
    """Eq. 10 + top-n on [B,H,T,nsel] (reference nsa/kernels.py:1965-2040).  Head sum
    in head order; ties resolved to the lower block index (stable sort)."""
    x = np.asarray(sel_scores)
    B, H, T, nsel = x.shape
    hpg = H // G
    agg = x.reshape(B, G, hpg, T, nsel)[:, :, 0].copy()
    for hh in range(1, hpg):
        agg = agg + x.reshape(B, G, hpg, T, nsel)[:, :, hh]
    order = np.argsort(-agg, axis=-1, kind="stable")
    k = min(n, nsel)
    top = order[..., :k]
    out = np.full((B, G, T, n), -1, dtype=np.int64)
    for b in range(B):
        for g in range(G):
            for t in range(T):
                cand = []
                if include_fixed and n_fixed > 0:
                    cand = [0, max(0, (t - lprime) // lprime), t // lprime]
                cand += top[b, g, t].tolist()
                seen = []
                for c in cand:
                    if c not in seen:
                        seen.append(c)
                    if len(seen) == n:
                        break
                out[b, g, t, :len(seen)] = seen
    return out


def _linear(x, w, b=None):
    y = x @ np.asarray(w, dtype=np.float64).T
    return y + np.asarray(b, dtype=np.float64) if b is not None else y


def compress_tokens(keys, values, w1, b1, w2, b2, pos_embed, l=32, d=16):
    """Reference compress_tokens (nsa/kernels.py:2119-2208) in float64.
    keys [B,G,T,dk], values [B,G,T,dv]; compress MLP Linear(dk+l,2dk)-ReLU-Linear(2dk,dk),
    pos_embed [l,l].  Returns (K_cmp [B,G,dk,NBp], V_cmp [B,G,NBp,dv], block_ends [NBp],
    n_actual), NBp the power-of-two padded count (padding: zeros, block_ends 999999)."""
    keys = np.asarray(keys, dtype=np.float64)
    values = np.asarray(values, dtype=np.float64)
    B, G, T, dk = keys.shape
    dv = values.shape[-1]
    n_act = (T - l) // d + 1
    n_pad = 1
    while n_pad < n_act:
        n_pad *= 2
    kc = np.zeros((B, G, dk, n_pad))
    vc = np.zeros((B, G, n_pad, dv))
    be = np.full((n_pad,), 999999, dtype=np.int32)
    pe = np.asarray(pos_embed, dtype=np.float64)
    for i in range(max(n_act, 0)):
        st = i * d
        en = min(st + l, T)
        blk = keys[:, :, st:en]
        x = np.concatenate([blk, np.broadcast_to(pe[: en - st], (B, G, en - st, l))], axis=-1)
        h = np.maximum(_linear(x, w1, b1), 0.0)
        y = _linear(h, w2, b2)
        kc[:, :, :, i] = y.mean(axis=2)
        vc[:, :, i] = values[:, :, st:en].mean(axis=2)
        be[i] = i * d + l - 1
    return kc, vc, be, n_act


def nsa_forward(x, params, cfg, indices=None):
    """NSAAttention forward (reference nsa/kernels.py:2210-2478) in float64 on numpy.

    params: dict of numpy weights keyed like the module's state_dict.  cfg: object with
    the NSAConfig fields.  Selection indices come from score_topn (fp32, the same
    pipeline the GPU runs) unless given.  Returns (out [B,T,D], info dict)."""
    x = np.asarray(x, dtype=np.float64)
    B, T, D = x.shape
    H, G, dk, dv = cfg.n_heads, cfg.n_kv_groups, cfg.head_dim_qk, cfg.head_dim_v
    P = {k: np.asarray(v, dtype=np.float64) for k, v in params.items()}

    def proj(name, heads, width):
        y = _linear(x, P[name + ".weight"], P.get(name + ".bias"))
        return y.reshape(B, T, heads, width).transpose(0, 2, 1, 3)

    q = proj("q_proj", H, dk)
    kcomp, vcomp = proj("k_compress", G, dk), proj("v_compress", G, dv)
    ksel, vsel = proj("k_select", G, dk), proj("v_select", G, dv)
    kslw, vslw = proj("k_sliding", G, dk), proj("v_sliding", G, dv)
    scale = 1.0 / math.sqrt(dk)
    kc, vc, be, _ = compress_tokens(kcomp, vcomp, P["compress_mlp.0.weight"], P.get("compress_mlp.0.bias"),
                                    P["compress_mlp.2.weight"], P.get("compress_mlp.2.bias"), P["pos_embed.weight"],
                                    cfg.l, cfg.d)
    if indices is None:
        indices = score_topn(q.astype(np.float32), kc.astype(np.float32), be, np.float32(scale), l=cfg.l, d=cfg.d,
                             lprime=cfg.l_prime, n=cfg.n, include_fixed=cfg.include_fixed_in_selection,
                             n_fixed=cfg.n_fixed)
    idx = np.asarray(indices, dtype=np.int64).copy()
    # the autograd wrapper's fallback: a row with no valid slot selects t // l'
    tb = (np.arange(T) // cfg.l_prime).reshape(1, 1, T, 1)
    no_valid = (idx < 0).all(axis=-1, keepdims=True)
    idx = np.where(no_valid, tb, idx)
    o_cmp, _, _ = attn_fwd(COMPRESSION, q, kc.transpose(0, 1, 3, 2), vc, scale, block_ends=be)
    o_sel, _, _ = attn_fwd(SELECTION, q, ksel, vsel, scale, indices=idx, lprime=cfg.l_prime)
    o_win, _, _ = attn_fwd(SLIDING, q, kslw, vslw, scale, window=cfg.w)
    h1 = np.maximum(_linear(x, P["gate_mlp.0.weight"], P.get("gate_mlp.0.bias")), 0.0)
    gl = _linear(h1, P["gate_mlp.2.weight"], P.get("gate_mlp.2.bias")).reshape(B, T, H, 3).transpose(0, 2, 1, 3)
    if cfg.gate_mode == "softmax":
        e = np.exp(gl - gl.max(-1, keepdims=True))
        gates = e / e.sum(-1, keepdims=True)
    else:
        gates = 1.0 / (1.0 + np.exp(-gl))
    mixed = o_cmp * gates[..., 0:1] + o_sel * gates[..., 1:2] + o_win * gates[..., 2:3]
    mixed = mixed.transpose(0, 2, 1, 3).reshape(B, T, H * dv)
    out = _linear(mixed, P["o_proj.weight"], P.get("o_proj.bias"))
    return out, {"selected_indices": indices, "gates": gates.transpose(0, 2, 1, 3), "k_cmp": kc, "v_cmp": vc,
                 "block_ends": be}


def dense_masked_attention(q, k, v, mask, scale):
    """Textbook dense formulation used to pin the per-row oracle:
    softmax((q k^T) * scale masked) v with GQA expansion; fully masked rows -> 0.
    q [B,H,Tq,dk], k [B,G,Tkv,dk], v [B,G,Tkv,dv], mask [B,H,Tq,Tkv] bool."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    H, G = q.shape[1], k.shape[1]
    ke = np.repeat(k, H // G, axis=1)
    ve = np.repeat(v, H // G, axis=1)
    s = np.einsum("bhtd,bhjd->bhtj", q, ke) * scale
    s = np.where(mask, s, -np.inf)
    mx = s.max(-1, keepdims=True)
    mx = np.where(np.isfinite(mx), mx, 0.0)
    e = np.where(mask, np.exp(s - mx), 0.0)
    den = e.sum(-1, keepdims=True)
    p = np.divide(e, den, out=np.zeros_like(e), where=den > 0)
    return np.einsum("bhtj,bhjd->bhtd", p, ve)
