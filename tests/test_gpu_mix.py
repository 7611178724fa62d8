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
