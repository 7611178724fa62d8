"""Randomised shapes (fixed seeds): every branch forward + backward against the oracle on
shapes drawn from the ranges the reference's launches allow -- batch, groups, heads per
group (1..20, including the 16-head groups of the stored-dS backward), ragged lengths,
every compiled head-dim pair and zero-padded widths below them, windows from 1 to past the
sequence, compression (l, d) pairs, selection block sizes (multiples of 16) and slot
counts with -1 padding and repeated blocks.  The drawn shape is printed before the GPU
runs it.  Tolerances as in test_gpu_branches.py: fp32 outputs 1e-5, gradients 1e-4;
bf16 2e-2 (the oracle fed the bf16-rounded inputs)."""
import math

import numpy as np
import pytest
import torch

import oracle
from conftest import rel_err
from nsa import _ops

pytestmark = pytest.mark.gpu

TOL = {torch.float32: (1e-5, 1e-4), torch.bfloat16: (2e-2, 2e-2)}
DIMS = [(32, 32), (48, 40), (64, 64), (100, 64), (128, 128), (192, 128)]


def _np(t):
    return t.detach().float().cpu().double().numpy()


def _draw(seed):
    rng = np.random.default_rng(seed)
    dtype = torch.bfloat16 if rng.random() < 0.5 else torch.float32
    G = int(rng.integers(1, 4))
    hpg = int(rng.choice([1, 2, 3, 4, 5, 16, 20]))
    B = int(rng.integers(1, 3))
    T = int(rng.integers(1, 400))
    dk, dv = DIMS[int(rng.integers(len(DIMS)))]
    kind = int(rng.integers(3))
    extra = {}
    if kind == _ops.SLIDING:
        extra["window"] = int(rng.choice([1, 2, 17, 64, 100, 300, 1000]))
    elif kind == _ops.COMPRESSION:
        l, d = [(32, 16), (16, 8), (8, 8), (32, 32)][int(rng.integers(4))]
        extra["ld"] = (l, d)
    else:
        extra["lprime"] = int(rng.choice([16, 32, 48, 64, 128]))
        extra["n"] = int(rng.integers(1, 17))
    return dict(kind=kind, dtype=dtype, B=B, G=G, H=G * hpg, T=T, dk=dk, dv=dv, extra=extra, seed=seed)


@pytest.mark.parametrize("seed", range(32))
def test_random_shape_parity(dev, seed):
    c = _draw(1000 + seed)
    print(f"[random] {c}", flush=True)
    kind, dtype, B, G, H, T, dk, dv = (c[k] for k in ("kind", "dtype", "B", "G", "H", "T", "dk", "dv"))
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, T, dk, generator=g).to(dtype)
    kw, okw = {}, {}
    Tkv = T
    if kind == _ops.SLIDING:
        kw["window"] = okw["window"] = c["extra"]["window"]
    elif kind == _ops.COMPRESSION:
        l, d = c["extra"]["ld"]
        n_act = max((T - l) // d + 1, 0)
        n_pad = 1 << max(n_act - 1, 0).bit_length()
        be = torch.full((n_pad,), 999999, dtype=torch.int32)
        be[:n_act] = torch.arange(n_act, dtype=torch.int32) * d + l - 1
        Tkv = n_pad
        kw["block_ends"], okw["block_ends"] = be.to(dev), be.numpy()
    else:
        lp, n = c["extra"]["lprime"], c["extra"]["n"]
        rng = np.random.default_rng(seed)
        idx = rng.integers(0, (T + lp - 1) // lp, size=(B, G, T, n))
        idx[rng.random(idx.shape) < 0.2] = -1
        if n > 1:
            idx[..., 1] = np.where(rng.random((B, G, T)) < 0.1, idx[..., 0], idx[..., 1])  # repeated blocks
        kw.update(indices=torch.tensor(idx, device=dev), lprime=lp)
        okw.update(indices=idx, lprime=lp)
    k = torch.randn(B, G, Tkv, dk, generator=g).to(dtype)
    v = torch.randn(B, G, Tkv, dv, generator=g).to(dtype)
    do = torch.randn(B, H, T, dv, generator=g).to(dtype)
    q, k, v, do = q.to(dev), k.to(dev), v.to(dev), do.to(dev)
    scale = 1 / math.sqrt(dk)
    out, L, M = _ops.attn_fwd(kind, q, k, v, scale, **kw)
    dq, dk_, dv_ = _ops.attn_bwd(kind, q, k, v, out, do, L, M, scale, **kw)
    torch.cuda.synchronize()
    ro, rL, rM = oracle.attn_fwd(kind, _np(q), _np(k), _np(v), scale, **okw)
    rq, rk, rv = oracle.attn_bwd(kind, _np(q), _np(k), _np(v), _np(do), scale, **okw)
    tol_o, tol_g = TOL[dtype]
    errs = {"out": rel_err(_np(out), ro), "dq": rel_err(_np(dq), rq), "dk": rel_err(_np(dk_), rk),
            "dv": rel_err(_np(dv_), rv)}
    # a reference tensor that is exactly zero (every row masked, or a window of one key,
    # where softmax is constant and dQ = dK = 0 up to the rounding of dP - D) must come
    # back zero to within that rounding
    for name, got, ref in (("out", out, ro), ("dq", dq, rq), ("dk", dk_, rk), ("dv", dv_, rv)):
        if not np.any(ref):
            assert got.abs().max().item() < (2e-2 if dtype == torch.bfloat16 else 1e-5), name
            errs[name] = 0.0
    print(f"[random] errors {errs}", flush=True)
    assert errs["out"] < tol_o and max(errs["dq"], errs["dk"], errs["dv"]) < tol_g, errs
    Ln, Mn = L.cpu().numpy(), M.cpu().numpy()
    assert np.array_equal(np.isneginf(Ln), np.isneginf(rL))
    fin = np.isfinite(rL)
    np.testing.assert_allclose(Ln[fin] + Mn[fin], rL[fin] + rM[fin], rtol=0,
                               atol=5e-3 if dtype == torch.bfloat16 else 2e-5)
