"""GPU tests of the NSAAttention module end to end: forward against the reference's
golden outputs (eval mode) and the oracle, gradients against float64 torch autograd
of the same computation, and the fused compress_tokens against the oracle."""
import math
import types

import numpy as np
import pytest
import torch

import oracle
import torch_nsa_ref
from conftest import load_fixture, rel_err
from nsa import NSAAttention, NSAConfig

pytestmark = pytest.mark.gpu


def _cfg_from(f):
    return NSAConfig(**{k[4:]: f[k].item() for k in f.files if k.startswith("cfg/")})


def _module_from(f, dev, dtype=torch.float32):
    cfg = _cfg_from(f)
    m = NSAAttention(cfg)
    m.load_state_dict({k[6:]: torch.tensor(f[k]) for k in f.files if k.startswith("param/")})
    return m.to(dev, dtype), cfg


@pytest.fixture(autouse=True)
def _ieee_fp32():
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    yield
    torch.backends.cuda.matmul.allow_tf32 = prev


@pytest.mark.parametrize("name", ["module_cfg1", "module_odd_softmax", "module_short"])
def test_module_forward_matches_reference_golden(dev, name):
    f = load_fixture(name)
    m, cfg = _module_from(f, dev)
    m.eval()
    with torch.no_grad():
        out, info = m(torch.tensor(f["x"]).to(dev), output_attentions=True)
    np.testing.assert_array_equal(info["selected_indices"].cpu().numpy(), f["selected_indices"])
    assert rel_err(out.cpu().numpy(), f["out"]) < 1e-5
    np.testing.assert_allclose(info["compression_scores"].cpu().numpy(), f["compression_scores"], rtol=0, atol=1e-5)
    np.testing.assert_allclose(info["selection_scores"].cpu().numpy(), f["selection_scores"], rtol=0, atol=1e-4)
    np.testing.assert_allclose(info["gates"].cpu().numpy(), f["gates"], rtol=0, atol=1e-6)
    # and the oracle's float64 restatement with the same weights and indices
    ro, _ = oracle.nsa_forward(f["x"], {k[6:]: f[k] for k in f.files if k.startswith("param/")}, cfg,
                               indices=info["selected_indices"].cpu().numpy())
    assert rel_err(out.cpu().numpy(), ro) < 1e-5


@pytest.mark.parametrize("gate_mode,fixed", [("sigmoid", True), ("softmax", False)])
def test_module_gradients_match_autograd(dev, gate_mode, fixed):
    torch.manual_seed(0)
    cfg = NSAConfig(d_model=64, head_dim_qk=64, head_dim_v=64, n_heads=8, n_kv_groups=2, l=32, d=16, l_prime=64,
                    n=4, w=96, gate_mode=gate_mode, include_fixed_in_selection=fixed, use_bias=True)
    m = NSAAttention(cfg).to(dev)
    B, T = 2, 333
    x = torch.randn(B, T, cfg.d_model, device=dev, requires_grad=True)
    out, info = m(x, output_attentions=True)
    gout = torch.randn_like(out)
    out.backward(gout)
    idx = info["selected_indices"].cpu()
    P = {k: v.detach().cpu().double().requires_grad_() for k, v in m.state_dict().items()}
    xr = x.detach().cpu().double().requires_grad_()
    ref = torch_nsa_ref.nsa_forward(xr, P, cfg, idx)
    ref.backward(gout.cpu().double())
    assert rel_err(out.detach().cpu().numpy(), ref.detach().numpy()) < 1e-5
    assert rel_err(x.grad.cpu().numpy(), xr.grad.numpy()) < 1e-3
    grads = dict(m.named_parameters())
    for k, p in P.items():
        g, r = grads[k].grad.cpu().numpy(), p.grad.numpy()
        if np.linalg.norm(r) < 1e-9 * np.sqrt(r.size):
            # biases of the selection / sliding keys shift every logit of a row
            # equally: the softmax is invariant, the exact gradient is 0
            assert np.abs(g).max() < 1e-5, k
            continue
        assert rel_err(g, r) < 1e-3, k


def test_module_bf16_matches_oracle(dev, monkeypatch):
    """The bf16 module at the paper head shape (dk 192, dv 128, 16 heads per group)
    against the oracle fed the module's own bf16 tensors: the scoring inputs it computed
    (q, K_cmp, block ends) must give bit-identical indices, and the attention core's
    output (three branches, sigmoid gates, gated mix) must match the float64 oracle on
    the same q / K / V / gate logits within the bf16 tolerance (2e-2)."""
    import nsa.kernels as K

    torch.manual_seed(1)
    cfg = NSAConfig(d_model=128, head_dim_qk=192, head_dim_v=128, n_heads=16, n_kv_groups=1, n=8, w=128)
    m = NSAAttention(cfg).to(dev, torch.bfloat16)
    B, T = 1, 512
    x = torch.randn(B, T, cfg.d_model, device=dev).to(torch.bfloat16).requires_grad_()
    cap = {}
    real_score, real_apply = K.score_and_select, K.NSACore.apply

    def score(q, kc, be, scale, c, return_scores=False):
        cap["score"] = (q.detach().clone(), kc.detach().clone(), be.clone(), scale)
        return real_score(q, kc, be, scale, c, return_scores=return_scores)

    def core(*args):
        cap["core"] = [a.detach().clone() if torch.is_tensor(a) else a for a in args]
        o = real_apply(*args)
        cap["out"] = o.detach().clone()
        return o

    monkeypatch.setattr(K, "score_and_select", score)
    monkeypatch.setattr(K.NSACore, "apply", core)
    out, info = m(x, output_attentions=True)
    out.float().sum().backward()
    assert torch.isfinite(x.grad.float()).all()

    def f(t):
        return t.float().cpu().numpy()

    q, kc, be, scale = cap["score"]
    ref_idx = oracle.score_topn(f(q), f(kc), be.cpu().numpy(), np.float32(scale), l=cfg.l, d=cfg.d,
                                lprime=cfg.l_prime, n=cfg.n, include_fixed=cfg.include_fixed_in_selection,
                                n_fixed=cfg.n_fixed)
    np.testing.assert_array_equal(info["selected_indices"].cpu().numpy(), ref_idx)

    qk, kcmp, vcmp, be2, ksel_t, vsel, idx, kwin_t, vwin, gl, sc, _ = cap["core"]
    idx = idx.cpu().numpy().astype(np.int64)
    # rows with no valid slot select their own block (the wrapper's fallback)
    tb = (np.arange(T) // cfg.l_prime).reshape(1, 1, T, 1)
    idx = np.where((idx < 0).all(axis=-1, keepdims=True), tb, idx)
    o_c = oracle.attn_fwd(oracle.COMPRESSION, f(qk), f(kcmp).transpose(0, 1, 3, 2), f(vcmp), sc,
                          block_ends=be2.cpu().numpy())[0]
    o_s = oracle.attn_fwd(oracle.SELECTION, f(qk), f(ksel_t).transpose(0, 1, 3, 2), f(vsel), sc, indices=idx,
                          lprime=cfg.l_prime)[0]
    o_w = oracle.attn_fwd(oracle.SLIDING, f(qk), f(kwin_t).transpose(0, 1, 3, 2), f(vwin), sc, window=cfg.w)[0]
    g = 1.0 / (1.0 + np.exp(-f(gl).astype(np.float64)))  # sigmoid gates [B,H,T,3]
    mixed = o_c * g[..., 0:1] + o_s * g[..., 1:2] + o_w * g[..., 2:3]
    assert rel_err(f(cap["out"]), mixed) < 2e-2


@pytest.mark.parametrize("T,dtype,token_major", [(512, torch.float32, False), (1000, torch.bfloat16, False),
                                                 (40, torch.float32, False), (1000, torch.bfloat16, True),
                                                 (40, torch.float32, True)])
def test_compress_tokens_matches_oracle(dev, T, dtype, token_major):
    """token_major: keys / values are [B,G,T,d] views of [B,T,G,d] storage (the module's
    projections), which the pooling kernels read in place."""
    torch.manual_seed(2)
    cfg = NSAConfig(d_model=64, head_dim_qk=64, head_dim_v=32, n_heads=4, n_kv_groups=2)
    m = NSAAttention(cfg).to(dev, dtype)
    keys = torch.randn(2, 2, T, 64, device=dev, dtype=dtype)
    vals = torch.randn(2, 2, T, 32, device=dev, dtype=dtype)
    if token_major:
        keys = keys.transpose(1, 2).contiguous().transpose(1, 2)
        vals = vals.transpose(1, 2).contiguous().transpose(1, 2)
    with torch.no_grad():
        kc, vc, be, n_act = m.compress_tokens(keys, vals)
    P = {k: v.float().cpu().numpy() for k, v in m.state_dict().items()}
    rk, rv, rbe, rn = oracle.compress_tokens(keys.float().cpu().numpy(), vals.float().cpu().numpy(),
                                             P["compress_mlp.0.weight"], P["compress_mlp.0.bias"],
                                             P["compress_mlp.2.weight"], P["compress_mlp.2.bias"],
                                             P["pos_embed.weight"], cfg.l, cfg.d)
    assert n_act == rn and kc.shape == rk.shape and vc.shape == rv.shape
    np.testing.assert_array_equal(be.cpu().numpy(), rbe)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert rel_err(kc.float().cpu().numpy(), rk) < tol
    assert rel_err(vc.float().cpu().numpy(), rv) < tol


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_compress_tokens_token_major_gradients(dev, dtype):
    """Gradients of compress_tokens through the token-major pooling path ([B,T,G,d]
    storage) equal those of the group-major path on the same values."""
    torch.manual_seed(5)
    cfg = NSAConfig(d_model=64, head_dim_qk=64, head_dim_v=32, n_heads=4, n_kv_groups=2)
    m = NSAAttention(cfg).to(dev, dtype)
    T = 300
    k0 = torch.randn(2, 2, T, 64, device=dev, dtype=dtype)
    v0 = torch.randn(2, 2, T, 32, device=dev, dtype=dtype)
    dk_out = dv_out = None
    grads = []
    for tm in (False, True):
        m.zero_grad()
        kl = (k0.transpose(1, 2).contiguous() if tm else k0.clone()).requires_grad_()
        vl = (v0.transpose(1, 2).contiguous() if tm else v0.clone()).requires_grad_()
        kc, vc, _, _ = m.compress_tokens(kl.transpose(1, 2) if tm else kl, vl.transpose(1, 2) if tm else vl)
        if dk_out is None:
            g = torch.Generator(device=dev).manual_seed(6)
            dk_out = torch.randn(kc.shape, device=dev, generator=g).to(dtype)
            dv_out = torch.randn(vc.shape, device=dev, generator=g).to(dtype)
        (kc.float() * dk_out.float()).sum().add((vc.float() * dv_out.float()).sum()).backward()
        gk = kl.grad.transpose(1, 2) if tm else kl.grad
        gv = vl.grad.transpose(1, 2) if tm else vl.grad
        grads.append([gk.float(), gv.float()] + [p.grad.float().clone() for p in m.parameters() if p.grad is not None])
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert len(grads[0]) == len(grads[1]) > 2
    for a, b in zip(*grads):
        assert rel_err(b.cpu().numpy(), a.cpu().numpy()) < tol


@pytest.mark.parametrize("rows,dtype", [(32768, torch.bfloat16), (4096, torch.float32), (300, torch.float32)])
def test_linear_split_k_gradients(dev, rows, dtype):
    """The compression MLP's linear layers reduce their weight gradient over every token
    in row chunks (one batched GEMM, fp32 partials): gradients against fp64 autograd."""
    from nsa.kernels import _LinearSplitK
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(2, rows // 2, 96, device=dev, generator=g).to(dtype).requires_grad_()
    W = (torch.randn(80, 96, device=dev, generator=g) * 0.1).to(dtype).requires_grad_()
    b = torch.randn(80, device=dev, generator=g).to(dtype).requires_grad_()
    dy = torch.randn(2, rows // 2, 80, device=dev, generator=g).to(dtype)
    _LinearSplitK.apply(x, W, b).backward(dy)
    xr, Wr, br = (t.detach().double().requires_grad_() for t in (x, W, b))
    torch.nn.functional.linear(xr, Wr, br).backward(dy.double())
    tol = 1e-2 if dtype == torch.bfloat16 else 1e-5
    for got, ref in ((x.grad, xr.grad), (W.grad, Wr.grad), (b.grad, br.grad)):
        assert rel_err(got.double().cpu().numpy(), ref.cpu().numpy()) < tol


@pytest.mark.parametrize("rows,n1,n2,pad", [(32768, 384, 192, 0), (2044, 192, 384, 0), (1000, 64, 128, 8),
                                            (65, 64, 64, 0), (63, 64, 64, 16), (1, 128, 64, 0), (0, 64, 64, 0)])
def test_wgrad_matches_fp64(dev, rows, n1, n2, pad):
    """nsa_wgrad (the bf16 weight gradient of the compression MLP's layers): dW = dY^T X
    against fp64 on the same bf16 inputs, within the bf16 rounding of the result; rows
    that do not fill a chunk or a 64-row step, padded row strides, no rows at all (zeros);
    two calls equal bit for bit."""
    from nsa import _lib, _ops
    g = torch.Generator(device=dev).manual_seed(rows + n1)
    dy = torch.randn(rows, n1 + pad, device=dev, generator=g).to(torch.bfloat16)[:, :n1]
    x = torch.randn(rows, n2 + pad, device=dev, generator=g).to(torch.bfloat16)[:, :n2]
    ws = torch.empty(max(_lib.size("nsa_wgrad_workspace_size", rows, n1, n2), 1), device=dev, dtype=torch.uint8)
    outs = []
    for _ in range(2):
        dW = torch.full((n1, n2), float("nan"), device=dev).to(torch.bfloat16)
        _lib.call("nsa_wgrad", _ops._ptr(dy), dy.stride(0), _ops._ptr(x), x.stride(0), rows, n1, n2, _ops._ptr(dW),
                  dW.stride(0), _lib.NSA_BF16, _ops._ptr(ws), ws.numel(), _ops._stream(dev))
        outs.append(dW)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    ref = dy.double().t() @ x.double()
    got = outs[0].double()
    if rows == 0:
        assert torch.count_nonzero(got) == 0
        return
    err = float((got - ref).norm() / ref.norm())
    assert err < 5e-3, err
    with pytest.raises(_lib.NSAKernelError):
        _lib.call("nsa_wgrad", _ops._ptr(dy), dy.stride(0), _ops._ptr(x), x.stride(0), rows, n1, n2, _ops._ptr(dW),
                  dW.stride(0), _lib.NSA_F32, _ops._ptr(ws), ws.numel(), _ops._stream(dev))


def test_linear_split_k_hip_weight_gradient(dev):
    """_LinearSplitK at the compression MLP's bf16 shapes (first layer: 32768 token rows,
    W 384 x 192) takes nsa_wgrad for dW: gradients against fp64 autograd."""
    from nsa.kernels import _LinearSplitK
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(1, 8192, 4, 192, device=dev, generator=g).to(torch.bfloat16).requires_grad_()
    W = (torch.randn(384, 192, device=dev, generator=g) * 0.05).to(torch.bfloat16).requires_grad_()
    dy = torch.randn(1, 8192, 4, 384, device=dev, generator=g).to(torch.bfloat16)
    _LinearSplitK.apply(x, W, None).backward(dy)
    xr, Wr = (t.detach().double().requires_grad_() for t in (x, W))
    torch.nn.functional.linear(xr, Wr).backward(dy.double())
    for got, ref in ((x.grad, xr.grad), (W.grad, Wr.grad)):
        assert rel_err(got.double().cpu().numpy(), ref.cpu().numpy()) < 1e-2


def test_linear_split_k_broadcast_gradient(dev):
    """An output gradient broadcast along the token rows (row stride 0, as a sum over a
    broadcast weight gives) does not meet nsa_wgrad's row layout: _LinearSplitK takes the
    batched GEMM for it, and the weight gradient still matches fp64 autograd."""
    from nsa.kernels import _LinearSplitK, _wgrad_hip
    g = torch.Generator(device=dev).manual_seed(6)
    x = torch.randn(2048, 192, device=dev, generator=g).to(torch.bfloat16).requires_grad_()
    W = (torch.randn(128, 192, device=dev, generator=g) * 0.05).to(torch.bfloat16).requires_grad_()
    dy = torch.randn(1, 128, device=dev, generator=g).to(torch.bfloat16).expand(2048, 128)
    assert not _wgrad_hip(dy, x.detach(), W)
    assert _wgrad_hip(dy.contiguous(), x.detach(), W)
    _LinearSplitK.apply(x, W, None).backward(dy)
    xr, Wr = (t.detach().double().requires_grad_() for t in (x, W))
    torch.nn.functional.linear(xr, Wr).backward(dy.double())
    assert rel_err(W.grad.double().cpu().numpy(), Wr.grad.cpu().numpy()) < 1e-2


def test_inference_mode_eval_then_training_step(dev):
    """An eval step under torch.inference_mode() first (it fills the module's cached
    block_ends), then a training step with the same shape: its backward saves that
    tensor and must run.  compress_tokens hands out its own copy of block_ends."""
    torch.manual_seed(3)
    cfg = NSAConfig(d_model=64, head_dim_qk=64, head_dim_v=64, n_heads=8, n_kv_groups=2, l=32, d=16, l_prime=64,
                    n=4, w=64)
    m = NSAAttention(cfg).to(dev)
    x = torch.randn(1, 333, cfg.d_model, device=dev)
    m.eval()
    with torch.inference_mode():
        ref, _ = m(x)
    m.train()
    xg = x.clone().requires_grad_(True)
    out, _ = m(xg)
    out.square().sum().backward()
    assert torch.isfinite(xg.grad).all() and rel_err(out.detach().cpu().numpy(), ref.cpu().numpy()) < 1e-5
    k = torch.randn(1, 2, 333, 64, device=dev)
    _, _, be1, _ = m.compress_tokens(k, k)
    be1.fill_(0)  # the caller's copy: later calls are unaffected
    _, _, be2, n_act = m.compress_tokens(k, k)
    assert be2[:n_act].tolist() == [i * 16 + 31 for i in range(n_act)]
