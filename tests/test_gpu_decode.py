"""GPU tests of the decode extensions (no counterpart in the reference): query rows placed
at an absolute position q_offset of the key sequence.

* Kernel level: the forward of each branch for rows r0.. of q with q_offset = r0 equals
  those rows of the full forward (the same keys, masks from absolute positions), and the
  Eq. 8 -> top-n scoring with q_offset gives bit-identical indices and scores.
* Module level: NSAAttention.prefill + decode one token at a time reproduces the rows of
  NSAAttention.forward over the whole sequence (the same weights, eval mode), and the
  CPU oracle: indices bit-exact to oracle.score_topn on the step's own query and cached
  compressed keys, outputs within 1e-5 (fp32) / 2e-2 (bf16) of oracle.nsa_forward.
"""
import math

import numpy as np
import pytest
import torch

from conftest import rel_err
from nsa import NSAAttention, NSAConfig, NSAKVCache, _ops
from nsa.kernels import score_and_select

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().double().numpy()


def _indices(seed, B, G, T, lp, n):
    g = torch.Generator().manual_seed(seed)
    nb = (T + lp - 1) // lp
    idx = torch.randint(0, nb, (B, G, T, n), generator=g)
    idx[torch.rand(B, G, T, n, generator=g) < 0.15] = -1
    return idx


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("r0", [0, 137, 299])
def test_branch_forward_with_q_offset(dev, dtype, r0):
    B, H, G, T, dk, dv, w, l, d, lp, n = 1, 8, 2, 300, 64, 64, 64, 32, 16, 32, 4
    g = torch.Generator().manual_seed(r0 + 1)
    q = torch.randn(B, H, T, dk, generator=g).to(dtype).to(dev)
    k = torch.randn(B, G, T, dk, generator=g).to(dtype).to(dev)
    v = torch.randn(B, G, T, dv, generator=g).to(dtype).to(dev)
    nb = (T - l) // d + 1
    kc = torch.randn(B, G, nb, dk, generator=g).to(dtype).to(dev)
    vc = torch.randn(B, G, nb, dv, generator=g).to(dtype).to(dev)
    be = (torch.arange(nb) * d + l - 1).to(torch.int32).to(dev)
    idx = _indices(r0, B, G, T, lp, n).to(dev)
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    qs = q[:, :, r0:].contiguous()
    cases = [
        (_ops.SLIDING, dict(window=w)),
        (_ops.COMPRESSION, dict(block_ends=be)),
        (_ops.SELECTION, dict(indices=idx, lprime=lp, fallback=True)),
    ]
    for kind, kw in cases:
        kk, vv = (kc, vc) if kind == _ops.COMPRESSION else (k, v)
        full, Lf, Mf = _ops.attn_fwd(kind, q, kk, vv, 0.125, **kw)
        kw2 = dict(kw)
        if kind == _ops.SELECTION:
            kw2["indices"] = idx[:, :, r0:]
        part, Lp, Mp = _ops.attn_fwd(kind, qs, kk, vv, 0.125, q_offset=r0, **kw2)
        torch.cuda.synchronize()
        assert rel_err(_np(part), _np(full[:, :, r0:])) < tol, kind
        fin = torch.isfinite(Lf[:, :, r0:])
        assert torch.equal(fin, torch.isfinite(Lp)), kind
        np.testing.assert_allclose(_np((Lp + Mp)[fin]), _np((Lf + Mf)[:, :, r0:][fin]), rtol=0,
                                   atol=5e-3 if dtype == torch.bfloat16 else 2e-5)


@pytest.mark.parametrize("r0", [1, 200, 511])
def test_score_topn_with_q_offset_bit_exact(dev, r0):
    B, H, G, T, dk, l, d, lp, n = 1, 8, 2, 512, 64, 32, 16, 64, 4
    g = torch.Generator().manual_seed(r0)
    q = torch.randn(B, H, T, dk, generator=g).to(dev)
    nb = (T - l) // d + 1
    n_pad = 1 << (nb - 1).bit_length()
    be = torch.full((n_pad,), 999999, dtype=torch.int32)
    be[:nb] = torch.arange(nb, dtype=torch.int32) * d + l - 1
    kc = torch.randn(B, G, dk, n_pad, generator=g).to(dev)
    cfg = NSAConfig(head_dim_qk=dk, n_heads=H, n_kv_groups=G, l=l, d=d, l_prime=lp, n=n)
    full = score_and_select(q, kc, be.to(dev), 1 / math.sqrt(dk), cfg, return_scores=True)
    part = score_and_select(q[:, :, r0:].contiguous(), kc, be.to(dev), 1 / math.sqrt(dk), cfg, return_scores=True,
                            q_offset=r0)
    for a, b in zip(part, full):
        assert torch.equal(a.cpu(), b[:, :, r0:].cpu())


@pytest.mark.parametrize("dtype,gate_mode", [(torch.float32, "sigmoid"), (torch.bfloat16, "softmax")])
def test_module_decode_matches_forward(dev, dtype, gate_mode):
    T, T0 = 200, 150
    cfg = NSAConfig(d_model=128, head_dim_qk=64, head_dim_v=64, n_heads=8, n_kv_groups=2, l=32, d=16, l_prime=32,
                    n=4, w=64, gate_mode=gate_mode)
    torch.manual_seed(0)
    m = NSAAttention(cfg).to(dev, dtype).eval()
    x = torch.randn(1, T, cfg.d_model, device=dev).to(dtype)
    with torch.no_grad():
        full, info = m(x, output_attentions=True)
    cache = NSAKVCache(cfg, 1, T, dev, dtype)
    m.prefill(x[:, :T0], cache)
    outs, sel = [], []
    for t in range(T0, T):
        o, inf = m.decode(x[:, t:t + 1], cache, output_attentions=True)
        outs.append(o)
        sel.append(inf["selected_indices"])
    dec = torch.cat(outs, dim=1)
    tol = 3e-2 if dtype == torch.bfloat16 else 1e-4
    assert rel_err(_np(dec), _np(full[:, T0:])) < tol
    assert cache.length == T and cache.n_act == (T - cfg.l) // cfg.d + 1


@pytest.mark.parametrize("dtype,gate_mode", [(torch.float32, "sigmoid"), (torch.bfloat16, "softmax")])
def test_module_decode_matches_oracle(dev, dtype, gate_mode):
    """Decode against the CPU oracle (the decode path has no reference counterpart; the
    forward it must reproduce row by row is nsa/kernels.py:2210-2478):
    * at every decoded position t, the selected indices equal oracle.score_topn on the
      module's own query row and the compressed keys cached at that step (the padded
      block count of that step), bit for bit;
    * the decoded outputs equal oracle.nsa_forward (float64 projections, compression,
      branches, gates and mix) at those rows, given the decoded indices: within 1e-5
      (fp32) and 2e-2 (bf16, the oracle fed the bf16 weights and input)."""
    import oracle
    T, T0 = 230, 100
    cfg = NSAConfig(d_model=128, head_dim_qk=64, head_dim_v=64, n_heads=8, n_kv_groups=2, l=32, d=16, l_prime=32,
                    n=5, w=48, gate_mode=gate_mode)
    torch.manual_seed(1)
    m = NSAAttention(cfg).to(dev, dtype).eval()
    x = torch.randn(1, T, cfg.d_model, device=dev).to(dtype)
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        cache = NSAKVCache(cfg, 1, T, dev, dtype)
        with torch.no_grad():
            m.prefill(x[:, :T0], cache)
            outs, sel = [], []
            for t in range(T0, T):
                o, inf = m.decode(x[:, t:t + 1], cache, output_attentions=True)
                outs.append(o)
                sel.append(inf["selected_indices"])
                # the query row and compressed keys this step scored with
                qt = m.q_proj(x[:, t:t + 1]).view(1, 1, cfg.n_heads, cfg.head_dim_qk).transpose(1, 2)
                n_pad = 1 << max(cache.n_act - 1, 0).bit_length()
                ridx = oracle.score_topn(_np(qt).astype(np.float32), _np(cache.K_cmp[..., :n_pad]).astype(np.float32),
                                         cache.block_ends[:n_pad].cpu().numpy(), np.float32(m.scale), l=cfg.l,
                                         d=cfg.d, lprime=cfg.l_prime, n=cfg.n, positions=np.array([t], np.int32))
                np.testing.assert_array_equal(inf["selected_indices"].cpu().numpy(), ridx, err_msg=f"t={t}")
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
    dec = _np(torch.cat(outs, dim=1))
    idx = torch.cat(sel, dim=2).cpu().numpy()
    # rows before T0 are not compared; any valid indices serve there
    full_idx = np.concatenate([np.zeros((1, cfg.n_kv_groups, T0, cfg.n), np.int64), idx], axis=2)
    params = {k_: _np(v_) for k_, v_ in m.state_dict().items()}
    ro, _ = oracle.nsa_forward(_np(x), params, cfg, indices=full_idx)
    err = rel_err(dec, ro[:, T0:])
    print(f"[decode] {dtype} vs oracle rel err {err:.2e}", flush=True)
    assert err < (2e-2 if dtype == torch.bfloat16 else 1e-5)
