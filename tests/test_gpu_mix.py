"""Fused gated mix (NSAAttention.forward, reference nsa/kernels.py:2446-2463) against a
float64 torch restatement of the same formula, forward and backward."""
import pytest
import torch

from conftest import rel_err as _rel


def rel_err(a, b):
    return _rel(a.detach().cpu().numpy(), b.detach().cpu().numpy())

pytestmark = pytest.mark.gpu


def _ref(o_c, o_s, o_w, g):
    return o_c * g[..., 0:1] + o_s * g[..., 1:2] + o_w * g[..., 2:3]


@pytest.mark.parametrize("B,H,T,dv,dtype", [(2, 4, 37, 64, torch.float32), (1, 8, 300, 128, torch.bfloat16),
                                            (1, 2, 5, 32, torch.bfloat16)])
def test_gated_mix_matches_formula(dev, B, H, T, dv, dtype):
    from nsa import GatedMix

    gen = torch.Generator(device="cpu").manual_seed(7)
    os_ = [torch.randn(B, H, T, dv, generator=gen).to(dev, dtype).requires_grad_() for _ in range(3)]
    # gates as the module makes them: a permuted view of [B, T, H, 3]
    logits = torch.randn(B, T, H, 3, generator=gen).to(dev, dtype)
    g = torch.sigmoid(logits).permute(0, 2, 1, 3).detach().requires_grad_()
    out = GatedMix.apply(*os_, g)
    assert out.shape == (B, H, T, dv)
    # [B,T,H,dv] storage: the module's transpose + reshape is free
    assert out.transpose(1, 2).is_contiguous()
    dout = torch.randn(B, T, H, dv, generator=gen).to(dev, dtype).transpose(1, 2)  # strided, as in the module
    out.backward(dout)

    r = [t.detach().double().requires_grad_() for t in os_]
    rg = g.detach().double().requires_grad_()
    ref = _ref(*r, rg)
    ref.backward(dout.double())
    tol = 1e-6 if dtype == torch.float32 else 8e-3
    assert rel_err(out.double(), ref) < tol
    for got, want in zip([t.grad for t in os_] + [g.grad], [t.grad for t in r] + [rg.grad]):
        assert rel_err(got.double(), want) < tol


@pytest.mark.parametrize("act", [0, 1, 2])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gate_activation_matches_torch(dev, act, dtype):
    """nsa_gate_act_fwd / _bwd (the fused path's gate activation and its gradient)
    against the torch fp32 formulas: the gate input is the module's [B,H,T,3] view of
    [B,T,H,3] storage; gates fp32 [3,B,H,T]; the input gradient in the input's dtype."""
    from nsa.kernels import _gate_activation, _gate_activation_grad
    B, H, T = 2, 5, 37
    g = torch.Generator().manual_seed(act)
    z = (torch.randn(B, T, H, 3, generator=g) * 3).to(dtype).to(dev).permute(0, 2, 1, 3)
    r = torch.randn(3, B, H, T, generator=g).to(dev)
    a = _gate_activation(z, act)
    dz = _gate_activation_grad(a, r, act, dtype)
    torch.cuda.synchronize()
    zf = z.double()
    ref = zf if act == 0 else torch.sigmoid(zf) if act == 1 else torch.softmax(zf, dim=-1)
    ref = ref.permute(3, 0, 1, 2)
    assert a.shape == (3, B, H, T) and a.dtype == torch.float32 and a.is_contiguous()
    assert (a.double() - ref).abs().max().item() < 2e-6
    ad, rd = a.double(), r.double()
    gref = rd if act == 0 else rd * ad * (1 - ad) if act == 1 else ad * (rd - (ad * rd).sum(0, keepdim=True))
    gref = gref.permute(1, 2, 3, 0)
    assert dz.shape == (B, H, T, 3) and dz.dtype == dtype
    assert _rel(dz.double().cpu().numpy(), gref.cpu().numpy()) < (1e-6 if dtype == torch.float32 else 1e-2)


@pytest.mark.parametrize("B,H,T,dv,dtype", [(1, 16, 300, 128, torch.bfloat16), (2, 4, 77, 64, torch.float32),
                                             (1, 8, 1000, 32, torch.bfloat16)])
def test_mix_row_dots(dev, B, H, T, dv, dtype):
    """nsa_mix_row_dots: dots[k] = sum_d dout . o_k for the three branch outputs, read in
    the module's [B,T,H,dv] storage, against float64 torch on the same values."""
    from nsa import _lib, _ops

    g = torch.Generator().manual_seed(7)
    ts = [torch.randn(B, T, H, dv, generator=g).to(dtype).to(dev).permute(0, 2, 1, 3) for _ in range(4)]
    d, o = ts[0], ts[1:]
    dots = torch.empty(3, B, H, T, device=dev, dtype=torch.float32)
    _lib.call("nsa_mix_row_dots", *[_ops._ptr(t) for t in ts], *d.stride()[:3], _ops._ptr(dots), B, H, T, dv,
              _ops._dtype_code(dtype), _ops._stream(dev))
    torch.cuda.synchronize()
    ref = torch.stack([(d.double() * x.double()).sum(-1) for x in o])
    assert _rel(dots.double().cpu().numpy(), ref.cpu().numpy()) < 1e-6
