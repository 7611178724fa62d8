"""The allocation-free sliding-window forward (nsa_sliding_window_fwd_noalloc, no
counterpart in the reference): called through the C ABI, it must give exactly what
nsa_sliding_window_fwd gives with a caller workspace (same kernels, bit for bit), on two
calls in a row with the second smaller (the static scratch keeps the first call's
contents), and refuse a shape beyond its 32 MiB scratch before launching anything."""
import ctypes
import math

import pytest
import torch

from nsa import _lib, _ops


def _call_noalloc(q, kp, v, out, L, M, scale, G, window, dtype_code, stream):
    B, H, T, dk = q.shape
    dv = v.shape[-1]
    P = ctypes.c_void_p
    return _lib.load().nsa_sliding_window_fwd_noalloc(
        P(q.data_ptr()), P(kp.data_ptr()), P(v.data_ptr()), P(out.data_ptr()), float(scale), P(L.data_ptr()),
        P(M.data_ptr()), *q.stride(), kp.stride(0), kp.stride(1), kp.stride(3), kp.stride(2), *v.stride(),
        *out.stride(), *L.stride(), *M.stride(), B, H, G, T, window, dk, dv, dtype_code, stream)


def test_noalloc_rejects_oversized_shape_before_launch():
    """Validation and the scratch limit are checked on the host first (no GPU needed)."""
    lib = _lib.load()
    need = _lib.size("nsa_fwd_workspace_size", 0, _lib.NSA_BF16, 1, 64, 8, 32768, 32768, 192, 128, 0, 64)
    assert need > 32 << 20
    rc = lib.nsa_sliding_window_fwd_noalloc(*([None] * 4), 1.0, None, None, *([0] * 22), 1, 64, 8, 32768, 512,
                                            192, 128, _lib.NSA_BF16, None)
    assert rc == _lib.NSA_ERR_WORKSPACE and b"static scratch" in lib.nsa_last_error()


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry_point(dev, dtype):
    code = _lib.NSA_BF16 if dtype == torch.bfloat16 else _lib.NSA_F32
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    # the first call fills most of the scratch (about 21 MB at the paper shape in bf16),
    # the second is smaller and must not see the first call's leftovers
    shapes = [(1, 64, 4, 8192, 192, 128, 512), (2, 8, 2, 1000, 64, 64, 100)]
    if dtype == torch.float32:
        shapes[0] = (1, 32, 4, 6000, 128, 128, 512)
    for i, (B, H, G, T, dk, dv, w) in enumerate(shapes):
        g = torch.Generator(device=dev).manual_seed(40 + i)
        q = torch.randn(B, H, T, dk, device=dev, generator=g).to(dtype)
        kp = torch.randn(B, G, dk, T, device=dev, generator=g).to(dtype)
        v = torch.randn(B, G, T, dv, device=dev, generator=g).to(dtype)
        scale = 1 / math.sqrt(dk)
        need = _lib.size("nsa_fwd_workspace_size", 0, code, B, H, G, T, T, dk, dv, 0, 64)
        assert need <= 32 << 20
        ref_o, ref_L, ref_M = _ops.attn_fwd(_ops.SLIDING, q, kp.transpose(-1, -2), v, scale, window=w)
        out = torch.full((B, H, T, dv), float("nan"), device=dev, dtype=dtype)
        L = torch.full((B, H, T), float("nan"), device=dev)
        M = torch.full((B, H, T), float("nan"), device=dev)
        print(f"[noalloc] call {i} shape B={B} H={H} G={G} T={T} dk={dk} dv={dv} w={w} {dtype}", flush=True)
        rc = _call_noalloc(q, kp, v, out, L, M, scale, G, w, code, stream)
        assert rc == 0, _lib.load().nsa_last_error()
        torch.cuda.synchronize()
        assert torch.equal(out, ref_o) and torch.equal(L, ref_L) and torch.equal(M, ref_M), i
