"""GPU parity of the fused Eq. 8 -> 9 -> 10 -> top-n kernel: selected block indices
bit-exact against the oracle (and the reference's golden vectors), and the optional
p_cmp / p_slc score tensors bit-exact too."""
import math

import numpy as np
import pytest
import torch

import oracle
from conftest import load_fixture
from nsa.kernels import NSAConfig, score_and_select

pytestmark = pytest.mark.gpu


def _block_ends(T, l, d):
    n_act = max((T - l) // d + 1, 0)
    n_pad = 1
    while n_pad < n_act:
        n_pad *= 2
    be = np.full(n_pad, 999999, dtype=np.int32)
    be[:n_act] = np.arange(n_act) * d + l - 1
    return be


def _run(dev, q, kc, be, scale, cfg, positions=None, want_scores=True):
    qd = torch.tensor(q).to(dev)
    kd = torch.tensor(kc).to(dev)
    bd = torch.tensor(be).to(dev)
    idx, pc, ps = score_and_select(qd, kd, bd, scale, cfg, return_scores=True)
    idx, pc, ps = idx.cpu().numpy(), pc.cpu().numpy(), ps.cpu().numpy()
    q32 = qd.float().cpu().numpy()
    k32 = kd.float().cpu().numpy()
    if positions is not None:
        q32 = q32[:, :, positions]
        idx, pc, ps = idx[:, :, positions], pc[:, :, positions], ps[:, :, positions]
    r = oracle.score_topn(q32, k32, be, np.float32(scale), l=cfg.l, d=cfg.d, lprime=cfg.l_prime, n=cfg.n,
                          include_fixed=cfg.include_fixed_in_selection, n_fixed=cfg.n_fixed, want_scores=want_scores,
                          positions=positions)
    return (idx, pc, ps), r


CASES = [
    # B, H, G, T, dk, l, d, l', n, include_fixed, dtype
    (1, 8, 2, 512, 64, 32, 16, 64, 4, True, torch.float32),      # benchmark config 1
    (2, 4, 2, 133, 32, 16, 8, 32, 3, False, torch.float32),
    (1, 4, 1, 24, 32, 32, 16, 64, 4, True, torch.float32),       # no compressed block visible anywhere
    (1, 16, 1, 700, 192, 32, 16, 64, 16, True, torch.bfloat16),
    (2, 8, 8, 300, 64, 32, 16, 64, 7, True, torch.float32),      # one head per group
    (1, 64, 1, 200, 32, 32, 16, 64, 5, True, torch.float32),     # 64 heads per group
]


@pytest.mark.parametrize("B,H,G,T,dk,l,d,lp,n,fixed,dtype", CASES)
def test_score_topn_bit_exact(dev, B, H, G, T, dk, l, d, lp, n, fixed, dtype):
    rng = np.random.default_rng(T + H)
    q = rng.standard_normal((B, H, T, dk)).astype(np.float32)
    be = _block_ends(T, l, d)
    kc = rng.standard_normal((B, G, dk, be.shape[0])).astype(np.float32)
    if dtype == torch.bfloat16:
        q = torch.tensor(q).to(torch.bfloat16).float().numpy()
        kc = torch.tensor(kc).to(torch.bfloat16).float().numpy()
    cfg = NSAConfig(head_dim_qk=dk, n_heads=H, n_kv_groups=G, l=l, d=d, l_prime=lp, n=n,
                    include_fixed_in_selection=fixed)
    qd = torch.tensor(q).to(dtype).to(dev)
    kd = torch.tensor(kc).to(dtype).to(dev)
    idx, pc, ps = (x.cpu().numpy() for x in score_and_select(qd, kd, torch.tensor(be).to(dev), 1 / math.sqrt(dk),
                                                             cfg, return_scores=True))
    ridx, rpc, rps = oracle.score_topn(q, kc, be, np.float32(1 / math.sqrt(dk)), l=l, d=d, lprime=lp, n=n,
                                       include_fixed=fixed, n_fixed=cfg.n_fixed, want_scores=True)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_array_equal(pc, rpc)
    np.testing.assert_array_equal(ps, rps)


@pytest.mark.parametrize("name", ["module_cfg1", "module_odd_softmax", "module_short", "heads_paper"])
def test_score_topn_golden(dev, name):
    """Indices of the reference module (eval mode) from its own q and K_cmp."""
    f = load_fixture(name)
    c = {k[4:]: f[k].item() for k in f.files if k.startswith("cfg/")}
    cfg = NSAConfig(**c)
    idx = score_and_select(torch.tensor(f["q"]).to(dev), torch.tensor(f["k_cmp"]).to(dev),
                           torch.tensor(f["block_ends"]).to(dev), 1 / math.sqrt(cfg.head_dim_qk), cfg)
    np.testing.assert_array_equal(idx.cpu().numpy(), f["selected_indices"])


def test_score_topn_tie_stress(dev):
    """Benchmark config 5: piecewise-constant keys per 64-token block make compressed
    scores tie exactly; early rows have fewer blocks than n (future blocks score 0 and
    are taken lowest index first).  Full size, fp32, bit-exact."""
    B, H, G, T, dk, l, d, lp, n = 4, 16, 4, 2048, 64, 32, 16, 64, 16
    rng = np.random.default_rng(55)
    blocks = rng.standard_normal((B, G, T // 64, dk)).astype(np.float32)
    k = np.repeat(blocks, 64, axis=2)  # [B,G,T,dk], constant over each 64-token block
    be = _block_ends(T, l, d)
    n_act = (T - l) // d + 1
    kc = np.zeros((B, G, dk, be.shape[0]), np.float32)
    for i in range(n_act):
        kc[:, :, :, i] = k[:, :, i * d:i * d + l].mean(axis=2)
    q = rng.standard_normal((B, H, T, dk)).astype(np.float32)
    cfg = NSAConfig(head_dim_qk=dk, n_heads=H, n_kv_groups=G, l=l, d=d, l_prime=lp, n=n)
    (idx, pc, ps), (ridx, rpc, rps) = _run(dev, q, kc, be, 1 / math.sqrt(dk), cfg)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_array_equal(ps, rps)
    # rows that see no compressed block score only block 0; the other slots are the
    # zero-score blocks in index order (stable sort), after de-duplication
    np.testing.assert_array_equal(idx[:, :, 0], np.broadcast_to(np.arange(n), (B, G, n)))
    assert (idx >= 0).all() and (idx < T // lp).all()


@pytest.mark.parametrize("cfgname", ["paper", "long"])
def test_score_topn_full_size_sampled(dev, cfgname):
    """Benchmark configs 3 and 4 at full size; the oracle checks a sample of rows
    (a row's indices depend only on its own queries and K_cmp)."""
    if cfgname == "paper":
        B, H, G, T, dk = 1, 64, 4, 8192, 192
    else:
        B, H, G, T, dk = 1, 32, 2, 32768, 128
    l, d, lp, n = 32, 16, 64, 16
    g = torch.Generator(device=dev).manual_seed(7)
    q = (torch.randn(B, H, T, dk, device=dev, generator=g) / math.sqrt(dk)).to(torch.bfloat16)
    be = _block_ends(T, l, d)
    kc = (torch.randn(B, G, dk, be.shape[0], device=dev, generator=g)).to(torch.bfloat16)
    cfg = NSAConfig(head_dim_qk=dk, n_heads=H, n_kv_groups=G, l=l, d=d, l_prime=lp, n=n)
    bd = torch.tensor(be).to(dev)
    idx = score_and_select(q, kc, bd, 1 / math.sqrt(dk), cfg).cpu().numpy()
    rows = np.unique(np.concatenate([np.arange(0, 40), np.linspace(0, T - 1, 40).astype(int), [T - 1]]))
    ridx = oracle.score_topn(q.float().cpu().numpy()[:, :, rows], kc.float().cpu().numpy(), be, np.float32(1 / math.sqrt(dk)),
                             l=l, d=d, lprime=lp, n=n, positions=rows)
    np.testing.assert_array_equal(idx[:, :, rows], ridx)
    # every row: block 0 first, the row's own block present, no repeats
    t = np.arange(T)
    np.testing.assert_array_equal(idx[..., 0], 0)
    assert (idx == (t // lp)[None, None, :, None]).any(-1).all()
    srt = np.sort(idx, axis=-1)
    assert not ((srt[..., 1:] == srt[..., :-1]) & (srt[..., 1:] >= 0)).any()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_score_topn_4096_columns_sampled(dev, dtype):
    """More than 2048 compressed blocks (T = 40000: 2499 blocks, rows of 2560 logits held
    as 16 pieces per lane).  Sampled rows, indices and scores bit-exact."""
    B, H, G, T, dk, l, d, lp, n = 1, 4, 2, 40000, 32, 32, 16, 64, 16
    g = torch.Generator(device=dev).manual_seed(11)
    q = (torch.randn(B, H, T, dk, device=dev, generator=g) / math.sqrt(dk)).to(dtype)
    be = _block_ends(T, l, d)
    kc = torch.randn(B, G, dk, be.shape[0], device=dev, generator=g).to(dtype)
    cfg = NSAConfig(head_dim_qk=dk, n_heads=H, n_kv_groups=G, l=l, d=d, l_prime=lp, n=n)
    idx, pc, ps = score_and_select(q, kc, torch.tensor(be).to(dev), 1 / math.sqrt(dk), cfg, return_scores=True)
    rows = np.unique(np.concatenate([np.arange(0, 20), np.linspace(0, T - 1, 30).astype(int), [T - 1]]))
    ridx, rpc, rps = oracle.score_topn(q.float().cpu().numpy()[:, :, rows], kc.float().cpu().numpy(), be,
                                       np.float32(1 / math.sqrt(dk)), l=l, d=d, lprime=lp, n=n, want_scores=True,
                                       positions=rows)
    np.testing.assert_array_equal(idx.cpu().numpy()[:, :, rows], ridx)
    np.testing.assert_array_equal(pc.cpu().numpy()[:, :, rows], rpc)
    np.testing.assert_array_equal(ps.cpu().numpy()[:, :, rows], rps)


@pytest.mark.parametrize("H,G,T,dk,dtype", [(64, 1, 9000, 32, torch.float32), (48, 2, 4500, 64, torch.bfloat16)])
def test_score_topn_multipass_sampled(dev, H, G, T, dk, dtype):
    """Many heads per group with many compressed blocks: a timestep's rows are scored
    in several LDS passes whose Eq. 10 sums continue in head order.  Sampled rows,
    indices and scores bit-exact."""
    B, l, d, lp, n = 1, 32, 16, 64, 16
    rng = np.random.default_rng(H + T)
    q = rng.standard_normal((B, H, T, dk)).astype(np.float32)
    be = _block_ends(T, l, d)
    kc = rng.standard_normal((B, G, dk, be.shape[0])).astype(np.float32)
    if dtype == torch.bfloat16:
        q = torch.tensor(q).to(torch.bfloat16).float().numpy()
        kc = torch.tensor(kc).to(torch.bfloat16).float().numpy()
    cfg = NSAConfig(head_dim_qk=dk, n_heads=H, n_kv_groups=G, l=l, d=d, l_prime=lp, n=n)
    qd = torch.tensor(q).to(dtype).to(dev)
    kd = torch.tensor(kc).to(dtype).to(dev)
    idx, pc, ps = (x.cpu().numpy() for x in score_and_select(qd, kd, torch.tensor(be).to(dev), 1 / math.sqrt(dk),
                                                             cfg, return_scores=True))
    rows = np.unique(np.concatenate([np.arange(0, 20), np.linspace(0, T - 1, 24).astype(int), [T - 1]]))
    ridx, rpc, rps = oracle.score_topn(q[:, :, rows], kc, be, np.float32(1 / math.sqrt(dk)), l=l, d=d, lprime=lp,
                                       n=n, positions=rows, want_scores=True)
    np.testing.assert_array_equal(idx[:, :, rows], ridx)
    np.testing.assert_array_equal(pc[:, :, rows], rpc)
    np.testing.assert_array_equal(ps[:, :, rows], rps)
