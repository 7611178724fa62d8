"""GPU parity of the three HIP attention branches (forward and backward) against the
CPU oracle, on the same seeded inputs.

Tolerances (norm-relative): fp32 outputs 1e-5, fp32 gradients 1e-4 (target 1e-3);
bf16 outputs and gradients 2e-2, with the oracle fed the bf16-rounded inputs.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from conftest import rel_err
from nsa import _ops
from nsa.kernels import (NSAConfig, SelectionAttention, _nsa_compression_bwd_kernel, _nsa_compression_fwd_kernel,
                         _nsa_sliding_window_bwd_kernel, _nsa_sliding_window_fwd_kernel,
                         _nsa_sparse_selection_bwd_kernel, _nsa_sparse_selection_fwd_kernel)

pytestmark = pytest.mark.gpu

TOL = {torch.float32: (1e-5, 1e-4), torch.bfloat16: (2e-2, 2e-2)}


def _np(t):
    return t.detach().float().cpu().double().numpy()


def _make(seed, B, H, G, Tq, Tkv, dk, dv, dtype, dev):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, Tq, dk, generator=g).to(dtype)
    kp = torch.randn(B, G, dk, Tkv, generator=g).to(dtype)  # reference layout [B,G,dk,T]
    v = torch.randn(B, G, Tkv, dv, generator=g).to(dtype)
    do = torch.randn(B, H, Tq, dv, generator=g).to(dtype)
    return q.to(dev), kp.to(dev), v.to(dev), do.to(dev)


def _check(kind, q, kp, v, do, scale, dtype, **kw):
    """Run fwd + bwd through the tensor-level wrappers and compare with the oracle."""
    k = kp.transpose(-1, -2)
    out, L, M = _ops.attn_fwd(kind, q, k, v, scale, **kw)
    dq, dk, dv = _ops.attn_bwd(kind, q, k, v, out, do, L, M, scale, **kw)
    torch.cuda.synchronize()
    okw = {key: (val.cpu().numpy() if torch.is_tensor(val) else val) for key, val in kw.items() if key != "fallback"}
    ro, rL, rM = oracle.attn_fwd(kind, _np(q), _np(k), _np(v), scale, **okw)
    rq, rk, rv = oracle.attn_bwd(kind, _np(q), _np(k), _np(v), _np(do), scale, **okw)
    tol_o, tol_g = TOL[dtype]
    errs = {"out": rel_err(_np(out), ro), "dq": rel_err(_np(dq), rq), "dk": rel_err(_np(dk), rk),
            "dv": rel_err(_np(dv), rv)}
    assert errs["out"] < tol_o and max(errs["dq"], errs["dk"], errs["dv"]) < tol_g, errs
    # statistics: -inf exactly where the oracle row is empty, close elsewhere
    Ln, Mn = L.cpu().numpy(), M.cpu().numpy()
    assert np.array_equal(np.isneginf(Ln), np.isneginf(rL))
    fin = np.isfinite(rL)
    np.testing.assert_allclose(Ln[fin] + Mn[fin], rL[fin] + rM[fin], rtol=0, atol=5e-3 if dtype == torch.bfloat16 else 2e-5)
    return out, (dq, dk, dv)


SLIDING_CASES = [
    # B, H, G, T, dk, dv, window, dtype
    (1, 8, 2, 512, 64, 64, 256, torch.float32),   # benchmark config 1 shape
    (2, 8, 2, 64, 32, 32, 16, torch.float32),     # reference tests/test_accuracy.py shape
    (1, 16, 1, 300, 192, 128, 100, torch.bfloat16),
    (2, 4, 4, 129, 64, 64, 512, torch.float32),   # window longer than the sequence
    (1, 4, 2, 77, 128, 128, 1, torch.float32),    # window 1: out = v_t
    (1, 8, 2, 700, 128, 128, 512, torch.bfloat16),
    (1, 6, 3, 96, 48, 48, 40, torch.float32),     # head dims zero-padded to a compiled pair
    (1, 6, 2, 333, 64, 64, 70, torch.bfloat16),   # 3 heads per group (not a power of two)
    # bf16 with whole 16-head groups: dQ from the dS the dK/dV kernel stores
    (1, 64, 2, 300, 64, 64, 40, torch.bfloat16),  # two head groups, a window shorter than a tile
    (2, 16, 1, 457, 128, 128, 200, torch.bfloat16),  # ragged T, window not a multiple of 32
]


@pytest.mark.parametrize("B,H,G,T,dk,dv,w,dtype", SLIDING_CASES)
def test_sliding_parity(dev, B, H, G, T, dk, dv, w, dtype):
    q, kp, v, do = _make(1, B, H, G, T, T, dk, dv, dtype, dev)
    if w > 1:
        _check(_ops.SLIDING, q, kp, v, do, 1 / math.sqrt(dk), dtype, window=w)
        return
    # window 1 (closed form): out = v_t, dV = sum of dO over the group's heads, and the
    # softmax is constant so dQ = dK = 0 up to fp32 rounding of dP - D
    k = kp.transpose(-1, -2)
    out, L, M = _ops.attn_fwd(_ops.SLIDING, q, k, v, 0.1, window=1)
    dq, dk_, dv_ = _ops.attn_bwd(_ops.SLIDING, q, k, v, out, do, L, M, 0.1, window=1)
    hpg = H // G
    torch.testing.assert_close(out, v.repeat_interleave(hpg, 1), rtol=0, atol=0)
    torch.testing.assert_close(dv_, do.view(B, G, hpg, T, dv).sum(2), rtol=1e-6, atol=1e-6)
    assert dq.abs().max().item() < 1e-5 and dk_.abs().max().item() < 1e-5


COMPRESSION_CASES = [
    # B, H, G, T, dk, dv, l, d, dtype
    (1, 8, 2, 512, 64, 64, 32, 16, torch.float32),
    (2, 8, 2, 64, 32, 32, 8, 8, torch.float32),
    (1, 16, 1, 1100, 192, 128, 32, 16, torch.bfloat16),
    (1, 4, 2, 20, 64, 64, 32, 16, torch.float32),  # no row sees a block: all zero, L = -inf
    (1, 4, 1, 5000, 128, 128, 32, 16, torch.bfloat16),
    (1, 6, 2, 400, 64, 64, 32, 16, torch.bfloat16),  # 3 heads per group
    (1, 32, 1, 777, 64, 64, 32, 16, torch.bfloat16),  # stored dS, two head groups, ragged T
]


@pytest.mark.parametrize("B,H,G,T,dk,dv,l,d,dtype", COMPRESSION_CASES)
def test_compression_parity(dev, B, H, G, T, dk, dv, l, d, dtype):
    n_act = max((T - l) // d + 1, 0)
    n_pad = 1
    while n_pad < max(n_act, 1):
        n_pad *= 2
    be = torch.full((n_pad,), 999999, dtype=torch.int32)
    be[:n_act] = torch.arange(n_act, dtype=torch.int32) * d + l - 1
    q, kp, v, do = _make(2, B, H, G, T, n_pad, dk, dv, dtype, dev)
    _check(_ops.COMPRESSION, q, kp, v, do, 1 / math.sqrt(dk), dtype, block_ends=be.to(dev))


def _random_indices(seed, B, G, T, Tkv, lp, n, p_empty=0.15):
    rng = np.random.default_rng(seed)
    nb = (Tkv + lp - 1) // lp
    idx = rng.integers(0, nb, size=(B, G, T, n))
    idx[rng.random(idx.shape) < p_empty] = -1
    return torch.tensor(idx)


SELECTION_CASES = [
    # B, H, G, T, dk, dv, l', n, dtype
    (1, 8, 2, 512, 64, 64, 64, 4, torch.float32),
    (2, 8, 2, 64, 32, 32, 16, 8, torch.float32),   # reference tests/test_selection_reference.py shape
    (2, 8, 2, 64, 32, 32, 32, 4, torch.float32),   # reference tests/test_branches.py shape
    (1, 16, 1, 700, 192, 128, 64, 16, torch.bfloat16),
    (1, 4, 1, 300, 64, 64, 128, 3, torch.float32),  # selection blocks larger than a tile
    (4, 16, 4, 256, 64, 64, 64, 16, torch.float32),  # n larger than the number of blocks
    (1, 32, 2, 1024, 128, 128, 64, 16, torch.bfloat16),
    (1, 2, 2, 400, 64, 64, 32, 16, torch.bfloat16),  # one head per group, 16 slots
    (1, 6, 2, 333, 64, 64, 48, 5, torch.float32),    # 3 heads per group, blocks straddling 32-key chunks
    # bf16 with whole 16-head groups: dQ from the dS the dK/dV kernel stores
    (1, 64, 2, 300, 64, 64, 64, 8, torch.bfloat16),   # two head groups per KV group
    (1, 16, 1, 500, 128, 128, 128, 4, torch.bfloat16),  # two 64-key sub-blocks per block
    (2, 32, 2, 200, 32, 32, 64, 16, torch.bfloat16),  # n larger than the number of blocks
    # bf16 with whole 16-head groups but l' not a multiple of 64: the recomputing dQ kernel
    (1, 16, 1, 500, 64, 64, 32, 8, torch.bfloat16),
]


@pytest.mark.parametrize("B,H,G,T,dk,dv,lp,n,dtype", SELECTION_CASES)
def test_selection_parity(dev, B, H, G, T, dk, dv, lp, n, dtype):
    q, kp, v, do = _make(3, B, H, G, T, T, dk, dv, dtype, dev)
    idx = _random_indices(4, B, G, T, T, lp, n)
    idx[0, 0, 1, :] = 0  # repeated block in one row: counted once
    _check(_ops.SELECTION, q, kp, v, do, 1 / math.sqrt(dk), dtype, indices=idx.to(dev), lprime=lp)


OVERWRITE_CASES = [
    # kind, B, H, G, Tq, Tkv, d, extra
    ("sliding_direct", 64, 8, 4, 256, 256, 64, dict(window=100)),  # items store their own keys
    ("sliding", 1, 8, 2, 700, 700, 64, dict(window=512)),          # partials + reduce
    ("compression", 1, 8, 2, 400, 32, 64, {}),
    ("selection", 1, 8, 2, 512, 512, 64, dict(lprime=64)),         # blocks 4.. never selected
    ("compression_empty", 1, 4, 2, 0, 16, 64, {}),                 # no query rows
    ("sliding_empty", 1, 4, 2, 0, 64, 64, dict(window=16)),        # no query rows
    ("selection_empty", 1, 4, 2, 0, 256, 64, dict(lprime=64)),     # no query rows
    ("selection_allneg", 1, 8, 2, 256, 256, 64, dict(lprime=64)),  # every slot -1: no row sees a key
    ("selection_noslots", 1, 8, 2, 256, 256, 64, dict(lprime=64)),  # n = 0 slots
]


@pytest.mark.parametrize("case,B,H,G,Tq,Tkv,d,extra", OVERWRITE_CASES)
def test_dkdv_overwrite_matches_accumulate(dev, case, B, H, G, Tq, Tkv, d, extra):
    """The backward extensions' dK/dV overwrite bit (bwd_flags NSA_BWD_DKDV_OVERWRITE):
    caller buffers pre-filled with garbage are overwritten with exactly the gradients of
    the default call, and without the bit a buffer of ones receives exactly 1 + those
    gradients (fp32: the kernels add the same fp32 sums).  Covers the sliding direct
    mode, the reduce pass (including selection tiles no row selected, which must be
    written as zeros), launches with no query rows and selections with no valid slot
    or no slots at all (every element zero).  The overwrite buffers start as NaN, so an
    element no kernel writes cannot pass."""
    kind = {"sliding": _ops.SLIDING, "compression": _ops.COMPRESSION, "selection": _ops.SELECTION}[case.split("_")[0]]
    dtype = torch.float32
    kw = dict(extra)
    q, kp, v, do = _make(11, B, H, G, Tq, Tkv, d, d, dtype, dev)
    if kind == _ops.COMPRESSION:
        be = torch.full((Tkv,), 999999, dtype=torch.int32)
        n_act = Tkv - 4  # four padding blocks that no row sees
        be[:n_act] = torch.arange(n_act, dtype=torch.int32) * 16 + 31
        kw["block_ends"] = be.to(dev)
    if case == "selection_allneg":
        kw["indices"] = torch.full((B, G, Tq, 3), -1, dtype=torch.int64, device=dev)
    elif case == "selection_noslots":
        kw["indices"] = torch.empty((B, G, Tq, 0), dtype=torch.int64, device=dev)
    elif kind == _ops.SELECTION:
        kw["indices"] = _random_indices(5, B, G, Tq, 4 * 64, 64, 3, p_empty=0.0).to(dev)
    k = kp.transpose(-1, -2)
    print(f"[overwrite] {case} B={B} H={H} G={G} Tq={Tq} Tkv={Tkv}", flush=True)
    out, L, M = _ops.attn_fwd(kind, q, k, v, 1 / math.sqrt(d), **kw)
    _, gk, gv = _ops.attn_bwd(kind, q, k, v, out, do, L, M, 1 / math.sqrt(d), **kw)
    dk1 = torch.full((B, G, Tkv, d), float("nan"), device=dev)
    dv1 = torch.full((B, G, Tkv, d), float("nan"), device=dev)
    _ops.attn_bwd(kind, q, k, v, out, do, L, M, 1 / math.sqrt(d), dk=dk1, dv=dv1, dkdv_overwrite=True, **kw)
    dk2 = torch.ones(B, G, Tkv, d, device=dev)
    dv2 = torch.ones(B, G, Tkv, d, device=dev)
    _ops.attn_bwd(kind, q, k, v, out, do, L, M, 1 / math.sqrt(d), dk=dk2, dv=dv2, **kw)
    torch.cuda.synchronize()
    assert torch.equal(dk1, gk) and torch.equal(dv1, gv)
    assert torch.equal(dk2, 1 + gk) and torch.equal(dv2, 1 + gv)
    if kind == _ops.SELECTION:  # keys of blocks no row selected
        assert torch.count_nonzero(gk[:, :, 4 * 64:]) == 0 and torch.count_nonzero(gv[:, :, 4 * 64:]) == 0
    if Tq == 0 or case in ("selection_allneg", "selection_noslots"):
        assert torch.count_nonzero(gk) == 0 and torch.count_nonzero(gv) == 0


ROW_DOT_CASES = [
    # kind, H, G, dtype: bf16 with a whole 16-head group takes the stored-dS backward
    # (row statistics from row_stats_kernel), the others the recomputing dQ kernels
    # (row statistics from the dQ kernel)
    (_ops.SLIDING, 16, 1, torch.bfloat16), (_ops.SLIDING, 8, 2, torch.float32),
    (_ops.COMPRESSION, 16, 1, torch.bfloat16), (_ops.COMPRESSION, 8, 2, torch.float32),
    (_ops.SELECTION, 16, 1, torch.bfloat16), (_ops.SELECTION, 8, 2, torch.float32),
]


@pytest.mark.parametrize("kind,H,G,dtype", ROW_DOT_CASES)
def test_row_dot_and_row_gate(dev, kind, H, G, dtype):
    """The backward extensions' row_dot output (sum_d dOut * Out per row, written when no
    delta is passed) and row_gate input (the branch's output gradient is row_gate * dOut):
    row_dot against the row sums of the forward's Out and dOut, the gradients against the
    oracle's backward of the gated dOut."""
    B, T, dk, dv = 1, 260, 64, 64
    q, kp, v, do = _make(41, B, H, G, T, T, dk, dv, dtype, dev)
    k = kp.transpose(-1, -2)
    if kind == _ops.SLIDING:
        kw = dict(window=70)
    elif kind == _ops.COMPRESSION:
        nb = (T - 32) // 16 + 1
        k, v = k[:, :, :nb].contiguous(), v[:, :, :nb].contiguous()
        kw = dict(block_ends=(torch.arange(nb) * 16 + 31).to(torch.int32).to(dev))
    else:
        kw = dict(indices=_random_indices(42, B, G, T, T, 64, 5).to(dev), lprime=64)
    scale = 1 / math.sqrt(dk)
    gate = torch.rand(B, H, T, generator=torch.Generator().manual_seed(43)).to(dev)
    out, L, M = _ops.attn_fwd(kind, q, k, v, scale, **kw)
    row_dot = torch.full((B, H, T), float("nan"), device=dev)
    dq, dk_, dv_ = _ops.attn_bwd(kind, q, k, v, out, do, L, M, scale, row_gate=gate, row_dot=row_dot, **kw)
    torch.cuda.synchronize()
    want = (out.double() * do.double()).sum(-1)
    assert rel_err(_np(row_dot), _np(want)) < 1e-5
    okw = {key: (val.cpu().numpy() if torch.is_tensor(val) else val) for key, val in kw.items()}
    dog = _np(do) * _np(gate)[..., None]
    rq, rk, rv = oracle.attn_bwd(kind, _np(q), _np(k), _np(v), dog, scale, **okw)
    tol = TOL[dtype][1]
    errs = {"dq": rel_err(_np(dq), rq), "dk": rel_err(_np(dk_), rk), "dv": rel_err(_np(dv_), rv)}
    assert max(errs.values()) < tol, errs


def test_selection_int32_indices_and_noncausal(dev):
    B, H, G, T, d, lp = 1, 4, 2, 128, 32, 32
    q, kp, v, do = _make(5, B, H, G, T, T, d, d, torch.float32, dev)
    idx = _random_indices(6, B, G, T, T, lp, 3)
    _check(_ops.SELECTION, q, kp, v, do, 0.2, torch.float32, indices=idx.to(torch.int32).to(dev), lprime=lp)
    _check(_ops.SELECTION, q, kp, v, do, 0.2, torch.float32, indices=idx.to(dev), lprime=lp, causal=False)


def test_selection_wrapper_fallback(dev):
    """SelectionAttention: a row whose slots are all -1 attends to its own block t//l'
    (nsa/kernels.py:199-205)."""
    B, H, G, T, d, lp, n = 1, 4, 2, 128, 32, 32, 4
    q, kp, v, do = _make(7, B, H, G, T, T, d, d, torch.float32, dev)
    idx = _random_indices(8, B, G, T, T, lp, n)
    idx[:, :, ::5] = -1
    cfg = NSAConfig(head_dim_qk=d, head_dim_v=d, n_heads=H, n_kv_groups=G, l_prime=lp, n=n)
    qq, kk, vv = (t.clone().requires_grad_() for t in (q, kp, v))
    out = SelectionAttention.apply(qq, kk, vv, idx.to(dev), 0.3, cfg)
    out.backward(do)
    eff = idx.clone()
    allneg = (eff < 0).all(-1)
    eff[allneg] = (torch.arange(T).view(1, 1, T).expand_as(allneg)[allneg] // lp).unsqueeze(-1)
    k = kp.transpose(-1, -2)
    ro, _, _ = oracle.attn_fwd(oracle.SELECTION, _np(q), _np(k), _np(v), 0.3, indices=eff.numpy(), lprime=lp)
    rq, rk, rv = oracle.attn_bwd(oracle.SELECTION, _np(q), _np(k), _np(v), _np(do), 0.3, indices=eff.numpy(),
                                 lprime=lp)
    assert rel_err(_np(out), ro) < 1e-5
    assert rel_err(_np(qq.grad), rq) < 1e-4
    assert rel_err(_np(kk.grad.transpose(-1, -2)), rk) < 1e-4
    assert rel_err(_np(vv.grad), rv) < 1e-4


def test_backward_is_deterministic(dev):
    B, H, G, T, dk, dv = 1, 16, 2, 600, 64, 64
    q, kp, v, do = _make(9, B, H, G, T, T, dk, dv, torch.bfloat16, dev)
    k = kp.transpose(-1, -2)
    idx = _random_indices(10, B, G, T, T, 64, 6).to(dev)
    n_act = (T - 32) // 16 + 1
    be = (torch.arange(n_act, dtype=torch.int32) * 16 + 31).to(dev)
    kc, vc = k[:, :, :n_act].contiguous(), v[:, :, :n_act].contiguous()
    for kind, kk, vv, kw in ((_ops.SLIDING, k, v, dict(window=128)), (_ops.COMPRESSION, kc, vc, dict(block_ends=be)),
                             (_ops.SELECTION, k, v, dict(indices=idx, lprime=64))):
        out, L, M = _ops.attn_fwd(kind, q, kk, vv, 0.125, **kw)
        g1 = _ops.attn_bwd(kind, q, kk, vv, out, do, L, M, 0.125, **kw)
        g2 = _ops.attn_bwd(kind, q, kk, vv, out, do, L, M, 0.125, **kw)
        for a, b in zip(g1, g2):
            assert torch.equal(a, b), kind


# ------------------------------------------------------- the raw launch surface
def test_raw_sliding_launch_matches_reference_contract(dev):
    """tests/test_kernel_contracts.py:22-172 of the reference: K [B,G,dk,T] with
    swapped strides, dK allocated [B,G,T,dk] and accumulated, backward from the
    forward's L/M; wrong (unswapped) strides give a different result."""
    B, H, G, T, dk, dv, w = 1, 4, 2, 64, 32, 32, 16
    q, k, v, do = _make(11, B, H, G, T, T, dk, dv, torch.float32, dev)
    scale = 1 / math.sqrt(dk)
    out = torch.zeros(B, H, T, dv, device=dev)
    L = torch.zeros(B, H, T, device=dev)
    M = torch.zeros(B, H, T, device=dev)
    grid = lambda META: (triton_cdiv(T, META["BLOCK_M"]), B * H)  # noqa: E731
    _nsa_sliding_window_fwd_kernel[grid](
        q, k, v, out, scale, L, M, *q.stride(), k.stride(0), k.stride(1), k.stride(3), k.stride(2), *v.stride(),
        *out.stride(), *L.stride(), *M.stride(), Z=B, H=H, N_KV_GROUPS=G, N_CTX=T, WINDOW_SIZE=w, HEAD_DIM_QK=dk,
        HEAD_DIM_V=dv, BLOCK_M=32, BLOCK_N=32)
    dq = torch.zeros_like(q)
    dkb = torch.zeros(B, G, T, dk, device=dev)
    dvb = torch.zeros_like(v)
    _nsa_sliding_window_bwd_kernel[grid](
        q, k, v, out, do, scale, L, M, *q.stride(), k.stride(0), k.stride(1), k.stride(3), k.stride(2), *v.stride(),
        *out.stride(), *L.stride(), *M.stride(), dq, dkb, dvb, *dq.stride(), *dkb.stride(), *dvb.stride(), Z=B, H=H,
        N_KV_GROUPS=G, N_CTX=T, WINDOW_SIZE=w, HEAD_DIM_QK=dk, HEAD_DIM_V=dv, BLOCK_M=32, BLOCK_N=32)
    torch.cuda.synchronize()
    kt = k.transpose(-1, -2)
    ro, _, _ = oracle.attn_fwd(oracle.SLIDING, _np(q), _np(kt), _np(v), scale, window=w)
    rq, rk, rv = oracle.attn_bwd(oracle.SLIDING, _np(q), _np(kt), _np(v), _np(do), scale, window=w)
    assert rel_err(_np(out), ro) < 1e-5
    assert rel_err(_np(dq), rq) < 1e-4 and rel_err(_np(dkb), rk) < 1e-4 and rel_err(_np(dvb), rv) < 1e-4
    # dK is accumulated into (callers zero it): a second launch doubles it
    _nsa_sliding_window_bwd_kernel[grid](
        q, k, v, out, do, scale, L, M, *q.stride(), k.stride(0), k.stride(1), k.stride(3), k.stride(2), *v.stride(),
        *out.stride(), *L.stride(), *M.stride(), dq, dkb, dvb, *dq.stride(), *dkb.stride(), *dvb.stride(), Z=B, H=H,
        N_KV_GROUPS=G, N_CTX=T, WINDOW_SIZE=w, HEAD_DIM_QK=dk, HEAD_DIM_V=dv, BLOCK_M=32, BLOCK_N=32)
    assert rel_err(_np(dkb), 2 * rk) < 1e-4
    # a square K ([dk == T]) with unswapped strides stays in bounds but reads the transpose
    ks = torch.randn(B, G, 32, 32, device=dev)
    qs = q[:, :, :32, :].contiguous()
    vs = v[:, :, :32, :].contiguous()
    o1 = torch.zeros(B, H, 32, dv, device=dev)
    o2 = torch.zeros(B, H, 32, dv, device=dev)
    for o, ksd in ((o1, (ks.stride(3), ks.stride(2))), (o2, (ks.stride(2), ks.stride(3)))):
        _nsa_sliding_window_fwd_kernel[(1, B * H)](
            qs, ks, vs, o, scale, L, M, *qs.stride(), ks.stride(0), ks.stride(1), *ksd, *vs.stride(), *o.stride(),
            *L.stride(), *M.stride(), Z=B, H=H, N_KV_GROUPS=G, N_CTX=32, WINDOW_SIZE=8, HEAD_DIM_QK=32,
            HEAD_DIM_V=32, BLOCK_M=32, BLOCK_N=32)
    assert ((o1 - o2).abs() / (o1.abs() + 1e-8)).max().item() > 0.1


def triton_cdiv(a, b):
    return (a + b - 1) // b


def test_raw_compression_and_selection_launch(dev):
    B, H, G, T, d = 2, 8, 2, 64, 32
    q, k, v, do = _make(12, B, H, G, T, T, d, d, torch.float32, dev)
    scale = 1 / math.sqrt(d)
    # compression with 8 blocks of 8 (reference tests/test_branches.py:235-252)
    nb = 8
    kc = torch.randn(B, G, d, nb, device=dev)
    vc = torch.randn(B, G, nb, d, device=dev)
    be = (torch.arange(nb, dtype=torch.int32) * 8 + 7).to(dev)
    out = torch.zeros(B, H, T, d, device=dev)
    L = torch.zeros(B, H, T, device=dev)
    M = torch.zeros(B, H, T, device=dev)
    _nsa_compression_fwd_kernel[(2, B * H)](
        q, kc, vc, be, out, scale, L, M, *q.stride(), kc.stride(0), kc.stride(1), kc.stride(3), kc.stride(2),
        *vc.stride(), *out.stride(), *L.stride(), *M.stride(), Z=B, H=H, N_KV_GROUPS=G, N_CTX_Q=T, N_BLOCKS=nb,
        HEAD_DIM_QK=d, HEAD_DIM_V=d, BLOCK_M=32, BLOCK_N=32)
    dq = torch.zeros_like(q)
    dkc = torch.zeros(B, G, nb, d, device=dev)
    dvc = torch.zeros_like(vc)
    _nsa_compression_bwd_kernel[(2, B * H)](
        q, kc, vc, be, out, do, scale, L, M, *q.stride(), kc.stride(0), kc.stride(1), kc.stride(3), kc.stride(2),
        *vc.stride(), *out.stride(), *L.stride(), *M.stride(), dq, dkc, dvc, *dq.stride(), *dkc.stride(),
        *dvc.stride(), Z=B, H=H, N_KV_GROUPS=G, N_CTX_Q=T, N_BLOCKS=nb, HEAD_DIM_QK=d, HEAD_DIM_V=d, BLOCK_M=32,
        BLOCK_N=32)
    kct = kc.transpose(-1, -2)
    ro, _, _ = oracle.attn_fwd(oracle.COMPRESSION, _np(q), _np(kct), _np(vc), scale, block_ends=be.cpu().numpy())
    rq, rk, rv = oracle.attn_bwd(oracle.COMPRESSION, _np(q), _np(kct), _np(vc), _np(do), scale,
                                 block_ends=be.cpu().numpy())
    assert rel_err(_np(out), ro) < 1e-5
    assert max(rel_err(_np(dq), rq), rel_err(_np(dkc), rk), rel_err(_np(dvc), rv)) < 1e-4
    # selection with fixed-style indices (reference tests/test_branches.py:474-499), N_CTX_KV > N_CTX_Q
    lp, n = 32, 4
    Tkv = 96
    ks = torch.randn(B, G, d, Tkv, device=dev)
    vs = torch.randn(B, G, Tkv, d, device=dev)
    nbk = (Tkv + lp - 1) // lp
    idx = torch.full((B, G, T, n), -1, dtype=torch.int32)
    for t in range(T):
        loc = t // lp
        cand = []
        for c in (0, max(0, loc - 1), loc, min(loc + 1, nbk - 1)):
            if c not in cand:
                cand.append(c)
        idx[:, :, t, :len(cand)] = torch.tensor(cand[:n], dtype=torch.int32)
    idx = idx.to(dev)
    out = torch.zeros(B, H, T, d, device=dev)
    _nsa_sparse_selection_fwd_kernel[(2, B * H)](
        q, ks, vs, idx, out, scale, L, M, *q.stride(), ks.stride(0), ks.stride(1), ks.stride(3), ks.stride(2),
        *vs.stride(), *out.stride(), *idx.stride(), *L.stride(), *M.stride(), Z=B, H=H, N_KV_GROUPS=G, N_CTX_Q=T,
        N_CTX_KV=Tkv, N_BLOCKS=n, BLOCK_SIZE_SELECTION=lp, HEAD_DIM_QK=d, HEAD_DIM_V=d, BLOCK_M=32, BLOCK_N=32,
        IS_CAUSAL=True)
    dq = torch.zeros_like(q)
    dks = torch.zeros(B, G, Tkv, d, device=dev)
    dvs = torch.zeros_like(vs)
    _nsa_sparse_selection_bwd_kernel[(2, B * H)](
        q, ks, vs, idx, out, do, scale, L, M, *q.stride(), ks.stride(0), ks.stride(1), ks.stride(3), ks.stride(2),
        *vs.stride(), *out.stride(), *idx.stride(), *L.stride(), *M.stride(), dq, dks, dvs, *dq.stride(),
        *dks.stride(), *dvs.stride(), Z=B, H=H, N_KV_GROUPS=G, N_CTX_Q=T, N_CTX_KV=Tkv, N_BLOCKS=n,
        BLOCK_SIZE_SELECTION=lp, HEAD_DIM_QK=d, HEAD_DIM_V=d, BLOCK_M=32, BLOCK_N=32, IS_CAUSAL=True)
    kst = ks.transpose(-1, -2)
    ro, _, _ = oracle.attn_fwd(oracle.SELECTION, _np(q), _np(kst), _np(vs), scale, indices=idx.cpu().numpy(),
                               lprime=lp)
    rq, rk, rv = oracle.attn_bwd(oracle.SELECTION, _np(q), _np(kst), _np(vs), _np(do), scale,
                                 indices=idx.cpu().numpy(), lprime=lp)
    assert rel_err(_np(out), ro) < 1e-5
    assert max(rel_err(_np(dq), rq), rel_err(_np(dks), rk), rel_err(_np(dvs), rv)) < 1e-4


def test_strided_views(dev):
    """Non-contiguous q / v / out views and a K whose time axis is not unit-stride."""
    B, H, G, T, d = 1, 4, 2, 200, 64
    base = torch.randn(B, T, H, d, device=dev)
    q = base.transpose(1, 2)  # [B,H,T,d] with strided rows
    kbig = torch.randn(B, G, T, d + 8, device=dev)
    kp = kbig[..., :d].transpose(-1, -2)  # [B,G,d,T], time stride = d + 8
    v = torch.randn(B, G, T, 2 * d, device=dev)[..., ::2]
    do = torch.randn(B, H, T, d, device=dev)
    _check(_ops.SLIDING, q, kp, v, do, 0.125, torch.float32, window=50)


@pytest.mark.parametrize("dk,dtype,gate_mode,H,lp", [(64, torch.float32, "sigmoid", 8, 32),
                                                      (192, torch.bfloat16, "sigmoid", 8, 32),
                                                      (192, torch.bfloat16, "softmax", 32, 64),
                                                      (48, torch.float32, "softmax", 8, 32)])
def test_nsa_core_matches_separate_functions(dev, dk, dtype, gate_mode, H, lp):
    """NSACore (the module's three branches, gate activation and gated mix, with the branch backwards
    taking the mix's row sums and summing dQ in the dQ kernels) against
    CompressionAttention / SelectionAttention / SlidingWindowAttention and GatedMix
    applied separately (autograd summing dQ): same output, same gradients.  dk = 48 is
    zero-padded to a compiled head dim, which takes the summed-on-the-host dQ path; 16
    heads per group with l' = 64 (bf16) take the stored-dS backward, whose selection dQ
    adds into the running dQ through its LDS-staged rows."""
    from nsa import NSACore
    from nsa.kernels import CompressionAttention, GatedMix, SlidingWindowAttention
    B, G, T, dv, l, d, n, w = 1, 2, 300, 64, 32, 16, 4, 64
    g = torch.Generator().manual_seed(11)
    nb = (T - l) // d + 1
    q = torch.randn(B, H, T, dk, generator=g).to(dtype)
    kc = torch.randn(B, G, dk, nb, generator=g).to(dtype)
    vc = torch.randn(B, G, nb, dv, generator=g).to(dtype)
    be = (torch.arange(nb) * d + l - 1).to(torch.int32)
    ks = torch.randn(B, G, dk, T, generator=g).to(dtype)
    vs = torch.randn(B, G, T, dv, generator=g).to(dtype)
    kw = torch.randn(B, G, dk, T, generator=g).to(dtype)
    vw = torch.randn(B, G, T, dv, generator=g).to(dtype)
    gate_logits = torch.randn(B, H, T, 3, generator=g).to(dtype)
    idx = _random_indices(12, B, G, T, T, lp, n).to(dev)
    do = torch.randn(B, H, T, dv, generator=g).to(dtype).to(dev)
    cfg = NSAConfig(head_dim_qk=dk, head_dim_v=dv, n_heads=H, n_kv_groups=G, l=l, d=d, l_prime=lp, n=n, w=w,
                    gate_mode=gate_mode)
    scale = 1 / math.sqrt(dk)

    def leaves():
        return [t.to(dev).requires_grad_() for t in (q, kc, vc, ks, vs, kw, vw, gate_logits)]

    a = leaves()
    out_a = NSACore.apply(a[0], a[1], a[2], be.to(dev), a[3], a[4], idx, a[5], a[6], a[7], scale, cfg)
    out_a.backward(do)
    b = leaves()
    outs_b = (CompressionAttention.apply(b[0], b[1], b[2], be.to(dev), scale, cfg),
              SelectionAttention.apply(b[0], b[3], b[4], idx, scale, cfg),
              SlidingWindowAttention.apply(b[0], b[5], b[6], scale, w, cfg))
    gb = torch.softmax(b[7].float(), dim=-1) if gate_mode == "softmax" else torch.sigmoid(b[7].float())
    out_b = GatedMix.apply(*outs_b, gb.to(dtype) if dtype == torch.float32 else gb)
    out_b.backward(do)
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    assert rel_err(_np(out_a), _np(out_b)) < (1e-2 if dtype == torch.bfloat16 else 1e-6)
    for x, y in zip(a, b):
        assert rel_err(_np(x.grad), _np(y.grad)) < tol


@pytest.mark.parametrize("kind", [_ops.SLIDING, _ops.COMPRESSION, _ops.SELECTION])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_dq_accumulate_adds_to_running_sum(dev, kind, dtype):
    """dq_accumulate: the branch's dQ is added to the values already in dq (the module's
    branches share one dQ buffer).  bf16 with a whole 16-head group takes the stored-dS
    dQ kernels (selection: the running rows staged through LDS)."""
    B, H, G, T, dk, dv = 1, 16, 1, 200, 192, 128
    q, kp, v, do = _make(21, B, H, G, T, T, dk, dv, dtype, dev)
    k = kp.transpose(-1, -2)
    if kind == _ops.SLIDING:
        kw = dict(window=50)
    elif kind == _ops.COMPRESSION:
        nb = (T - 32) // 16 + 1
        k, v = k[:, :, :nb].contiguous(), v[:, :, :nb].contiguous()
        kw = dict(block_ends=(torch.arange(nb) * 16 + 31).to(torch.int32).to(dev))
    else:
        kw = dict(indices=_random_indices(22, B, G, T, T, 64, 4).to(dev), lprime=64, fallback=True)
    out, L, M = _ops.attn_fwd(kind, q, k, v, 0.1, **kw)
    dq0, _, _ = _ops.attn_bwd(kind, q, k, v, out, do, L, M, 0.1, **kw)
    run = torch.randn(q.shape, device=dev).to(dtype)
    dq = run.clone()
    _ops.attn_bwd(kind, q, k, v, out, do, L, M, 0.1, dq=dq, dq_accumulate=True, **kw)
    want = run.float() + dq0.float()
    tol = 1e-2 if dtype == torch.bfloat16 else 1e-6
    assert rel_err(_np(dq), want.cpu().numpy()) < tol


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_time_contiguous_k_with_ragged_length(dev, dtype):
    """K in the reference's [B,G,dk,T] layout as a time slice of a longer buffer (feature
    stride a multiple of 16 bytes, T not): the transposing re-pack reads the last
    partial 16-byte run of each feature element by element."""
    B, H, G, T, d = 1, 16, 1, 300, 64
    q, _, v, do = _make(31, B, H, G, T, T, d, d, dtype, dev)
    kbig = torch.randn(B, G, d, 312, generator=torch.Generator().manual_seed(32)).to(dtype).to(dev)
    kp = kbig[..., :T]
    _check(_ops.SLIDING, q, kp, v, do, 0.125, dtype, window=77)



PAIR_CASES = [
    # B, H, G, T, dk, dv, window, row gates, accumulate
    (1, 16, 1, 300, 192, 128, 64, False, False),
    (2, 32, 2, 517, 64, 64, 200, True, True),
    (1, 16, 1, 1000, 128, 128, 512, True, True),
]


@pytest.mark.parametrize("B,H,G,T,dk,dv,w,gated,acc", PAIR_CASES)
def test_paired_dense_dq(dev, B, H, G, T, dk, dv, w, gated, acc):
    """A compression backward with its dQ deferred, then the sliding-window backward that
    adds it in its own dQ pass (bf16, whole 16-head groups): dQ against the sum of the
    two branches' oracle dQ (plus the running sum when accumulating) and against the two
    separate calls; dK / dV of both branches bit-equal to the separate calls."""
    dt = torch.bfloat16
    q, kp, v, do = _make(31, B, H, G, T, T, dk, dv, dt, dev)
    k = kp.transpose(-1, -2)
    nb = (T - 32) // 16 + 1
    n_pad = 1 << (nb - 1).bit_length()
    be = torch.full((n_pad,), 999999, dtype=torch.int32)
    be[:nb] = torch.arange(nb, dtype=torch.int32) * 16 + 31
    be = be.to(dev)
    g = torch.Generator().manual_seed(32)
    kc = torch.randn(B, G, n_pad, dk, generator=g).to(dt).to(dev)
    vc = torch.randn(B, G, n_pad, dv, generator=g).to(dt).to(dev)
    assert _ops.dq_deferrable(_ops.COMPRESSION, q, kc, vc) and _ops.dq_deferrable(_ops.SLIDING, q, k, v, window=w)
    scale = 1 / math.sqrt(dk)
    oc, Lc, Mc = _ops.attn_fwd(_ops.COMPRESSION, q, kc, vc, scale, block_ends=be)
    ow, Lw, Mw = _ops.attn_fwd(_ops.SLIDING, q, k, v, scale, window=w)
    gates = [torch.rand(B, H, T, device=dev) + 0.5 if gated else None for _ in range(2)]
    run = torch.randn(q.shape, device=dev).to(dt) if acc else torch.zeros(q.shape, device=dev, dtype=dt)
    # separate calls
    dq_sep = run.clone()
    _, dkc0, dvc0 = _ops.attn_bwd(_ops.COMPRESSION, q, kc, vc, oc, do, Lc, Mc, scale, block_ends=be, dq=dq_sep,
                                  dq_accumulate=acc, row_gate=gates[0])
    _, dkw0, dvw0 = _ops.attn_bwd(_ops.SLIDING, q, k, v, ow, do, Lw, Mw, scale, window=w, dq=dq_sep,
                                  dq_accumulate=True, row_gate=gates[1])
    # deferred + paired
    dq = run.clone()
    pend = _ops.DeferredDq()
    _, dkc1, dvc1 = _ops.attn_bwd(_ops.COMPRESSION, q, kc, vc, oc, do, Lc, Mc, scale, block_ends=be, dq=dq,
                                  row_gate=gates[0], defer_dq=pend)
    torch.cuda.synchronize()
    assert torch.equal(dq, run)  # the deferred call leaves dq alone
    _, dkw1, dvw1 = _ops.attn_bwd(_ops.SLIDING, q, k, v, ow, do, Lw, Mw, scale, window=w, dq=dq,
                                  dq_accumulate=acc, row_gate=gates[1], pair=pend)
    torch.cuda.synchronize()
    for a, b in ((dkc0, dkc1), (dvc0, dvc1), (dkw0, dkw1), (dvw0, dvw1)):
        assert torch.equal(a, b)
    assert rel_err(_np(dq), _np(dq_sep)) < 1e-2
    # the oracle: each branch's dQ with its gated dO
    dos = [do if gt is None else (do.float() * gt.unsqueeze(-1)).to(dt) for gt in gates]
    rq_c, _, _ = oracle.attn_bwd(oracle.COMPRESSION, _np(q), _np(kc), _np(vc), _np(dos[0]), scale,
                                 block_ends=be.cpu().numpy())
    rq_w, _, _ = oracle.attn_bwd(oracle.SLIDING, _np(q), _np(k), _np(v), _np(dos[1]), scale, window=w)
    want = rq_c + rq_w + (_np(run) if acc else 0)
    err = rel_err(_np(dq), want)
    print(f"[pair] B={B} H={H} G={G} T={T} dk={dk} w={w} gated={gated} acc={acc} dq err {err:.2e}", flush=True)
    assert err < 2e-2


def test_nsa_core_paper_shape_matches_separate_functions(dev):
    """NSACore at the paper shape (B=1, H=64, G=4, T=8192, dk=192, dv=128, bf16, n=16,
    w=512): its fused backward (selection dQ written first, the compression dQ added in the
    sliding-window dQ pass) against the three branch functions and GatedMix applied
    separately, on every input's gradient."""
    from nsa import NSACore
    from nsa.kernels import CompressionAttention, GatedMix, SlidingWindowAttention
    B, H, G, T, dk, dv, l, d, n, w, lp = 1, 64, 4, 8192, 192, 128, 32, 16, 16, 512, 64
    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(13)
    nb = (T - l) // d + 1
    npad = 1 << (nb - 1).bit_length()

    def rnd(*s, scale=1.0):
        return (torch.randn(*s, device=dev, generator=g) * scale).to(bf)

    q = rnd(B, H, T, dk, scale=dk ** -0.5)
    kc = torch.zeros(B, G, dk, npad, device=dev, dtype=bf)
    kc[..., :nb] = rnd(B, G, dk, nb, scale=dk ** -0.5)
    vc = torch.zeros(B, G, npad, dv, device=dev, dtype=bf)
    vc[:, :, :nb] = rnd(B, G, nb, dv)
    be = torch.full((npad,), 999999, dtype=torch.int32, device=dev)
    be[:nb] = torch.arange(nb, device=dev, dtype=torch.int32) * d + l - 1
    ks, kw = rnd(B, G, dk, T, scale=dk ** -0.5), rnd(B, G, dk, T, scale=dk ** -0.5)
    vs, vw = rnd(B, G, T, dv), rnd(B, G, T, dv)
    gate_logits = rnd(B, H, T, 3)
    idx = _random_indices(14, B, G, T, T, lp, n).to(dev)
    do = rnd(B, H, T, dv, scale=dv ** -0.5)
    cfg = NSAConfig(head_dim_qk=dk, head_dim_v=dv, n_heads=H, n_kv_groups=G, l=l, d=d, l_prime=lp, n=n, w=w)
    scale = dk ** -0.5

    def leaves():
        return [t.clone().requires_grad_() for t in (q, kc, vc, ks, vs, kw, vw, gate_logits)]

    a = leaves()
    NSACore.apply(a[0], a[1], a[2], be, a[3], a[4], idx, a[5], a[6], a[7], scale, cfg).backward(do)
    b = leaves()
    outs_b = (CompressionAttention.apply(b[0], b[1], b[2], be, scale, cfg),
              SelectionAttention.apply(b[0], b[3], b[4], idx, scale, cfg),
              SlidingWindowAttention.apply(b[0], b[5], b[6], scale, w, cfg))
    GatedMix.apply(*outs_b, torch.sigmoid(b[7].float())).backward(do)
    torch.cuda.synchronize()
    errs = {name: rel_err(_np(x.grad), _np(y.grad))
            for name, x, y in zip(("q", "kc", "vc", "ks", "vs", "kw", "vw", "gates"), a, b)}
    print(f"[core paper] gradient errors vs separate functions {errs}", flush=True)
    # observed on MI355X: 3.9e-3 .. 4.6e-3 (gates 1.5e-5); bound about twice that
    assert max(errs.values()) < 1e-2, errs
