"""CPU tests pinning the oracle (the checker of the HIP path).

Each oracle function is checked against something independent of its own code:
golden vectors written by the reference implementation (tests/golden), known-answer
vectors from the reference's tests, closed forms, a textbook dense formulation and
torch autograd.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from conftest import load_fixture, rel_err


# ----------------------------------------------------------------------- exp32
def test_exp32_accuracy_and_flush():
    xs = np.concatenate([np.linspace(-64.0, 0.0, 20001, dtype=np.float32),
                         -np.logspace(-8, 1.8, 2000).astype(np.float32), np.float32([0.0, -0.0])])
    got = oracle.exp32(xs).astype(np.float64)
    ref = np.exp(xs.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got - ref) / ulp) <= 2.0
    assert oracle.exp32(np.float32([-64.01, -100.0, -np.inf])).tolist() == [0.0, 0.0, 0.0]
    assert oracle.exp32(np.float32([0.0]))[0] == 1.0


# ---------------------------------------------------------- attention forward
def _mask_sliding(T, w):
    t = np.arange(T)
    return (t[None, :] <= t[:, None]) & (t[None, :] > t[:, None] - w)


def _mask_compression(T, be):
    return np.asarray(be)[None, :] <= np.arange(T)[:, None]


def _mask_selection(idx, T, Tkv, lp, causal=True):
    B, G, Tq, n = idx.shape
    m = np.zeros((B, G, Tq, Tkv), dtype=bool)
    for b in range(B):
        for g in range(G):
            for t in range(Tq):
                for blk in idx[b, g, t]:
                    if blk >= 0:
                        m[b, g, t, blk * lp:min(blk * lp + lp, Tkv)] = True
    if causal:
        m &= np.arange(Tkv)[None, None, None, :] <= np.arange(Tq)[None, None, :, None]
    return m


def _inputs(rng, B, H, G, T, Tkv, dk, dv):
    return (rng.standard_normal((B, H, T, dk)), rng.standard_normal((B, G, Tkv, dk)),
            rng.standard_normal((B, G, Tkv, dv)))


@pytest.mark.parametrize("T,w", [(64, 16), (97, 40), (50, 200)])
def test_sliding_matches_dense(T, w):
    rng = np.random.default_rng(0)
    B, H, G, dk, dv = 2, 4, 2, 8, 6
    q, k, v = _inputs(rng, B, H, G, T, T, dk, dv)
    out, L, M = oracle.attn_fwd(oracle.SLIDING, q, k, v, 0.3, window=w)
    mask = np.broadcast_to(_mask_sliding(T, w), (B, H, T, T))
    np.testing.assert_allclose(out, oracle.dense_masked_attention(q, k, v, mask, 0.3), rtol=1e-12, atol=1e-12)
    # L and M: log-sum-exp split around the row maximum
    s = np.einsum("bhtd,bhjd->bhtj", q, np.repeat(k, H // G, 1)) * 0.3
    s = np.where(mask, s, -np.inf)
    np.testing.assert_allclose(M, s.max(-1), rtol=1e-12)
    np.testing.assert_allclose(L + M, np.log(np.exp(s - s.max(-1, keepdims=True)).sum(-1)) + s.max(-1), rtol=1e-12)


def test_sliding_closed_forms():
    rng = np.random.default_rng(1)
    B, H, G, T, d = 1, 2, 1, 33, 4
    q, k, v = _inputs(rng, B, H, G, T, T, d, d)
    # window 1: every query sees only itself -> out = v_t
    out, _, _ = oracle.attn_fwd(oracle.SLIDING, q, k, v, 1.0, window=1)
    np.testing.assert_allclose(out, np.repeat(v, H, 1), rtol=1e-13)
    # window >= T: plain causal softmax attention
    out, _, _ = oracle.attn_fwd(oracle.SLIDING, q, k, v, 0.5, window=T)
    causal = np.tril(np.ones((T, T), dtype=bool))
    np.testing.assert_allclose(out, oracle.dense_masked_attention(q, k, v, np.broadcast_to(causal, (B, H, T, T)), 0.5),
                               rtol=1e-12)


def test_compression_matches_dense_and_empty_rows():
    rng = np.random.default_rng(2)
    B, H, G, T, nb, dk, dv = 1, 4, 2, 80, 5, 8, 8
    q, k, v = _inputs(rng, B, H, G, T, nb, dk, dv)
    be = np.arange(nb, dtype=np.int32) * 16 + 31
    out, L, M = oracle.attn_fwd(oracle.COMPRESSION, q, k, v, 0.25, block_ends=be)
    mask = np.broadcast_to(_mask_compression(T, be), (B, H, T, nb))
    np.testing.assert_allclose(out, oracle.dense_masked_attention(q, k, v, mask, 0.25), rtol=1e-12, atol=1e-12)
    # rows before the first block end see nothing: 0 output, L = M = -inf (nsa/reference.py:140-141)
    assert np.all(out[:, :, :31] == 0) and np.all(np.isneginf(L[:, :, :31])) and np.all(np.isneginf(M[:, :, :31]))
    assert np.all(np.isfinite(L[:, :, 31:]))


def test_selection_union_and_repeats():
    rng = np.random.default_rng(3)
    B, H, G, T, lp, n, d = 2, 4, 2, 96, 16, 4, 8
    q, k, v = _inputs(rng, B, H, G, T, T, d, d)
    idx = rng.integers(-1, T // lp, size=(B, G, T, n))
    idx[0, 0, 5] = [0, 0, 0, 0]  # a repeated block counts once
    idx[1, 1, 7] = [-1, -1, -1, -1]  # no block: empty row
    out, L, _ = oracle.attn_fwd(oracle.SELECTION, q, k, v, 0.4, indices=idx, lprime=lp)
    mask = np.repeat(_mask_selection(idx, T, T, lp), H // G, axis=1)
    np.testing.assert_allclose(out, oracle.dense_masked_attention(q, k, v, mask, 0.4), rtol=1e-12, atol=1e-12)
    assert np.isneginf(L[1, 2, 7]) and np.all(out[1, 2, 7] == 0)
    # non-causal mode sees the whole selected blocks
    out_nc, _, _ = oracle.attn_fwd(oracle.SELECTION, q, k, v, 0.4, indices=idx, lprime=lp, causal=False)
    mask_nc = np.repeat(_mask_selection(idx, T, T, lp, causal=False), H // G, axis=1)
    np.testing.assert_allclose(out_nc, oracle.dense_masked_attention(q, k, v, mask_nc, 0.4), rtol=1e-12, atol=1e-12)


def test_row_subset_positions():
    rng = np.random.default_rng(4)
    B, H, G, T, d = 1, 2, 1, 70, 4
    q, k, v = _inputs(rng, B, H, G, T, T, d, d)
    full, _, _ = oracle.attn_fwd(oracle.SLIDING, q, k, v, 0.5, window=9)
    rows = np.array([3, 40, 69])
    sub, _, _ = oracle.attn_fwd(oracle.SLIDING, q[:, :, rows], k, v, 0.5, window=9, positions=rows)
    np.testing.assert_array_equal(sub, full[:, :, rows])


# --------------------------------------------------------- attention backward
def _torch_dense_grads(q, k, v, do, mask, scale):
    qt, kt, vt = (torch.tensor(a, requires_grad=True) for a in (q, k, v))
    H, G = q.shape[1], k.shape[1]
    ke = kt.repeat_interleave(H // G, 1)
    ve = vt.repeat_interleave(H // G, 1)
    s = (qt @ ke.transpose(-1, -2)) * scale
    s = s.masked_fill(~torch.tensor(np.ascontiguousarray(mask)), float("-inf"))
    p = torch.softmax(s, -1).nan_to_num(0.0)
    (p @ ve).backward(torch.tensor(do))
    return qt.grad.numpy(), kt.grad.numpy(), vt.grad.numpy()


@pytest.mark.parametrize("kind", [oracle.SLIDING, oracle.COMPRESSION, oracle.SELECTION])
def test_backward_matches_autograd(kind):
    rng = np.random.default_rng(10 + kind)
    B, H, G, T, dk, dv = 2, 4, 2, 64, 8, 4
    kw = {}
    if kind == oracle.SLIDING:
        Tkv = T
        kw["window"] = 20
        mask = np.broadcast_to(_mask_sliding(T, 20), (B, H, T, T))
    elif kind == oracle.COMPRESSION:
        Tkv = 3
        be = np.arange(Tkv, dtype=np.int32) * 16 + 31
        kw["block_ends"] = be
        mask = np.broadcast_to(_mask_compression(T, be), (B, H, T, Tkv))
    else:
        Tkv = T
        idx = rng.integers(-1, T // 16, size=(B, G, T, 3))
        kw.update(indices=idx, lprime=16)
        mask = np.repeat(_mask_selection(idx, T, T, 16), H // G, axis=1)
    q, k, v = _inputs(rng, B, H, G, T, Tkv, dk, dv)
    do = rng.standard_normal((B, H, T, dv))
    dq, dk_, dv_ = oracle.attn_bwd(kind, q, k, v, do, 0.35, **kw)
    rq, rk, rv = _torch_dense_grads(q, k, v, do, mask, 0.35)
    for a, b in ((dq, rq), (dk_, rk), (dv_, rv)):
        np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-12)


# ------------------------------------------------------------ selection (Eq. 8-11)
def test_topn_known_answers():
    """Known-answer vectors of tests/test_whitepaper_spec.py:39-78 (reference)."""
    T, H, G, nb = 3, 2, 1, 5
    scores = np.broadcast_to(np.arange(nb, dtype=np.float32), (1, H, T, nb))
    idx = oracle.select_topk(scores, G, 3, 2, include_fixed=False, n_fixed=0)
    assert all(idx[0, 0, t].tolist() == [4, 3, 2] for t in range(T))
    idx = oracle.select_topk(scores, G, 3, 2, include_fixed=True, n_fixed=3)
    assert idx[0, 0, 0].tolist() == [0, 4, 3]
    assert idx[0, 0, 2].tolist() == [0, 1, 4]
    pad = oracle.select_topk(np.zeros((1, 2, 2, 2), np.float32), 1, 4, 2, include_fixed=True, n_fixed=3)
    assert pad.shape[-1] == 4 and (pad[0, 0, 0, 2:] == -1).all()


def test_eq9_first_block_closed_form():
    """p_slc[0] = p0 + 2 p1 + 2 p2 + 2 p3 + p4 for l/d = 2, l'/d = 4
    (the +m+n index of nsa/kernels.py:1956, cf. tests/test_comprehensive.py:146-154)."""
    rng = np.random.default_rng(5)
    p = rng.random((1, 1, 1, 12)).astype(np.float64)
    s = oracle.derive_selection(p)
    assert s.shape[-1] == 3
    np.testing.assert_allclose(s[..., 0], p[..., 0] + 2 * p[..., 1] + 2 * p[..., 2] + 2 * p[..., 3] + p[..., 4])
    np.testing.assert_allclose(s[..., 2], p[..., 8] + 2 * (p[..., 9] + p[..., 10] + p[..., 11]))


@pytest.mark.parametrize("name", ["topn_ties_fixed", "topn_ties_nofixed", "topn_causal_nexceeds"])
def test_topn_golden(name):
    g = load_fixture(name)
    G, n, lp, inc, nf = (int(x) for x in g["meta"])
    np.testing.assert_array_equal(oracle.select_topk(g["scores"], G, n, lp, bool(inc), nf), g["indices"])


def test_eq9_golden():
    g = load_fixture("eq9_random")
    np.testing.assert_array_equal(oracle.derive_selection(g["p_cmp"]), g["p_slc"])


MODULE_CASES = ["module_cfg1", "module_odd_softmax", "module_short"]


class _Cfg:
    def __init__(self, f):
        for k in f.files:
            if k.startswith("cfg/"):
                setattr(self, k[4:], f[k].item())


def _params(f):
    return {k[6:]: f[k] for k in f.files if k.startswith("param/")}


@pytest.mark.parametrize("name", MODULE_CASES)
def test_score_pipeline_golden(name):
    f = load_fixture(name)
    cfg = _Cfg(f)
    # Eq. 9 and Eq. 10/top-n on the reference's own scores: bit-exact
    np.testing.assert_array_equal(oracle.derive_selection(f["compression_scores"], cfg.l, cfg.d, cfg.l_prime),
                                  f["selection_scores"])
    np.testing.assert_array_equal(
        oracle.select_topk(f["selection_scores"], cfg.n_kv_groups, cfg.n, cfg.l_prime,
                           cfg.include_fixed_in_selection, cfg.n_fixed), f["selected_indices"])
    # the fp32 pipeline from q and K_cmp reproduces the reference's scores and indices
    idx, pc, ps = oracle.score_topn(f["q"], f["k_cmp"], f["block_ends"], np.float32(1 / math.sqrt(cfg.head_dim_qk)),
                                    l=cfg.l, d=cfg.d, lprime=cfg.l_prime, n=cfg.n,
                                    include_fixed=cfg.include_fixed_in_selection, n_fixed=cfg.n_fixed,
                                    want_scores=True)
    np.testing.assert_allclose(pc, f["compression_scores"], rtol=0, atol=2e-6)
    np.testing.assert_allclose(ps, f["selection_scores"], rtol=0, atol=2e-5)
    np.testing.assert_array_equal(idx, f["selected_indices"])


def test_score_pipeline_golden_paper_heads():
    """The reference module's selection at the paper's head shapes (dk = 192, 16 query
    heads per group, fp32): the oracle's fixed-order fp32 pipeline gives the same indices,
    and Eq. 9 scores within a few ulp of torch's matmul / softmax order."""
    f = load_fixture("heads_paper")
    cfg = _Cfg(f)
    idx, _, ps = oracle.score_topn(f["q"], f["k_cmp"], f["block_ends"], np.float32(1 / math.sqrt(cfg.head_dim_qk)),
                                   l=cfg.l, d=cfg.d, lprime=cfg.l_prime, n=cfg.n,
                                   include_fixed=cfg.include_fixed_in_selection, n_fixed=cfg.n_fixed,
                                   want_scores=True)
    np.testing.assert_allclose(ps, f["selection_scores"], rtol=4e-6, atol=0)
    np.testing.assert_array_equal(idx, f["selected_indices"])


@pytest.mark.parametrize("name", MODULE_CASES)
def test_compress_tokens_golden(name):
    f = load_fixture(name)
    cfg = _Cfg(f)
    P = _params(f)
    kc, vc, be, n_act = oracle.compress_tokens(f["k_comp_in"], f["v_comp_in"], P["compress_mlp.0.weight"],
                                               P["compress_mlp.0.bias"], P["compress_mlp.2.weight"],
                                               P["compress_mlp.2.bias"], P["pos_embed.weight"], cfg.l, cfg.d)
    assert n_act == int(f["n_actual"])
    np.testing.assert_array_equal(be, f["block_ends"])
    np.testing.assert_allclose(kc, f["k_cmp"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(vc, f["v_cmp"], rtol=0, atol=1e-6)


@pytest.mark.parametrize("name", MODULE_CASES)
def test_module_forward_golden(name):
    f = load_fixture(name)
    cfg = _Cfg(f)
    out, info = oracle.nsa_forward(f["x"], _params(f), cfg)
    np.testing.assert_array_equal(info["selected_indices"], f["selected_indices"])
    assert rel_err(out, f["out"]) < 1e-5
    np.testing.assert_allclose(info["gates"], f["gates"], rtol=0, atol=1e-6)
