"""Native Sparse Attention on MI355X: configuration, launch surface, autograd and module.

Drop-in for the reference's ``nsa.kernels`` (Noumena-Network/NSA-Test,
nsa/kernels.py).  Same public names and argument contracts:

* ``NSAConfig`` (nsa/kernels.py:516-591), including ``gate_mode`` and the
  ``include_fixed_in_selection`` / ``n_fixed`` normalisation;
* the six launchable kernels ``_nsa_{sliding_window,compression,sparse_selection}_
  {fwd,bwd}_kernel``, called as ``KERNEL[grid](*tensors_and_strides, **constexprs)``
  with the reference's positional order (nsa/kernels.py:594-654, :836-906,
  :1151-1191, :1303-1363, :1533-1574, :1690-1751), the [B,G,dk,T] K layout with
  swapped strides and the [B,G,T,dk] dK layout;
* the autograd wrappers ``CompressionAttention``, ``SelectionAttention``,
  ``SlidingWindowAttention`` (nsa/kernels.py:34-513);
* ``derive_selection_from_compression_per_timestep`` and
  ``select_top_k_blocks_per_query_with_gqa`` (nsa/kernels.py:1920-2040);
* ``NSAAttention`` (nsa/kernels.py:2043-2507) with the same sub-module names, so
  state dicts are interchangeable.

Every kernel runs in libnsa_hip.so (hand-written HIP for gfx950).  There is no CPU
path: tensors must live on the GPU, and a missing library raises.

Deliberate differences from the reference, all toward its own oracle
(nsa/reference.py):
* the compression wrapper reads K_cmp with the documented swapped strides (the
  reference wrapper passes them unswapped, nsa/kernels.py:62-65);
* head widths that are not powers of two (dk = 192) are handled exactly (the
  reference's sliding / compression launches read past the row, :85-86, :418-419);
* a block index repeated in one row counts once (the union of nsa/reference.py:
  233-246; the reference kernel visits it once per slot);
* Eq. 8 scores are computed in fp32 whatever the module dtype, and the eval path
  runs the same GPU kernels as training (they are deterministic) instead of
  float64 CPU loops (nsa/kernels.py:2366-2398).
"""
from __future__ import annotations

import functools
import math
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F

from . import _lib, _ops
from ._ops import COMPRESSION, SELECTION, SLIDING


# =============================================================================== config
@dataclass
class NSAConfig:
    """NSA hyper-parameters (paper section 4.1); field-for-field the reference's
    NSAConfig (nsa/kernels.py:516-591)."""

    d_model: int = 2560
    head_dim_qk: int = 192
    head_dim_v: int = 128
    l: int = 32
    d: int = 16
    l_prime: int = 64
    n: int = 16
    include_fixed_in_selection: bool = True
    n_fixed: int = 3
    n_dynamic: int = 13
    w: int = 512
    n_heads: int = 64
    n_kv_groups: int = 4
    dropout_p: float = 0.0
    use_bias: bool = False
    block_m: int = 32  # accepted for compatibility; the HIP kernels choose their own tiles
    block_n: int = 32
    gate_mode: str = "sigmoid"

    def __post_init__(self):
        assert self.n_heads % self.n_kv_groups == 0
        assert self.l % self.d == 0
        assert self.l_prime % self.d == 0
        assert self.w > 0
        if not self.include_fixed_in_selection:
            self.n_fixed = 0
        self.n_dynamic = max(0, self.n - self.n_fixed)
        assert self.n_fixed + self.n_dynamic == self.n
        assert self.gate_mode in ("sigmoid", "softmax")

    @property
    def heads_per_group(self) -> int:
        return self.n_heads // self.n_kv_groups

    @property
    def head_dim_qk_padded(self) -> int:
        p = 1
        while p < self.head_dim_qk:
            p *= 2
        return p

    @property
    def head_dim_v_padded(self) -> int:
        p = 1
        while p < self.head_dim_v:
            p *= 2
        return p


# ================================================================ launchable kernels
def _view(t, size, stride):
    """The logical tensor a Triton kernel would address: element x at
    base + sum(x_i * stride_i).  torch checks the view stays inside t's storage."""
    if t is None:
        return None
    return torch.as_strided(t, size, stride, t.storage_offset())


class _HipKernel:
    """``KERNEL[grid](*args, **constexprs)`` front end of one libnsa_hip.so entry point.

    The grid is accepted (tuple or callable of the meta-parameters) and ignored: the
    HIP kernels pick their own decomposition.  BLOCK_M / BLOCK_N are hints and
    HEAD_DIM_* may be padded widths; the real widths come from the tensors."""

    def __init__(self, name: str, branch: int, backward: bool):
        self.__name__ = name
        self.branch = branch
        self.backward = backward

    def __repr__(self):
        return f"<HIP kernel {self.__name__}>"

    def __getitem__(self, grid):
        if not (callable(grid) or isinstance(grid, (tuple, list))):
            raise TypeError("grid must be a tuple or a callable of the meta-parameters")
        return functools.partial(self._launch, grid)

    def _launch(self, grid, *args, **kw):
        br, bwd = self.branch, self.backward
        a = list(args)
        pos = 0

        def take(n):
            nonlocal pos
            out = a[pos:pos + n]
            pos += n
            return out

        if br == SLIDING:
            Q, K, V, Out = take(4)
            Blk = None
        elif br == COMPRESSION:
            Q, K, V, Blk, Out = take(5)
        else:
            Q, K, V, Blk, Out = take(5)
        dOut = take(1)[0] if bwd else None
        scale, L, M = take(3)
        sq, sk, sv, so = take(4), take(4), take(4), take(4)
        sb = take(4) if br == SELECTION else None
        sl, sm = take(3), take(3)
        if bwd:
            dQ, dK, dV = take(3)
            sdq, sdk, sdv = take(4), take(4), take(4)
        if pos != len(a):
            raise TypeError(f"{self.__name__}: expected {pos} positional arguments, got {len(a)}")
        Z, H, G = int(kw["Z"]), int(kw["H"]), int(kw["N_KV_GROUPS"])
        if br == SLIDING:
            Tq = Tkv = int(kw["N_CTX"])
        elif br == COMPRESSION:
            Tq, Tkv = int(kw["N_CTX_Q"]), int(kw["N_BLOCKS"])
        else:
            Tq, Tkv = int(kw["N_CTX_Q"]), int(kw["N_CTX_KV"])
        dk, dv = Q.shape[-1], V.shape[-1]
        q = _view(Q, (Z, H, Tq, dk), sq)
        k = _view(K, (Z, G, Tkv, dk), sk)
        v = _view(V, (Z, G, Tkv, dv), sv)
        o = _view(Out, (Z, H, Tq, dv), so)
        Lv = _view(L, (Z, H, Tq), sl)
        Mv = _view(M, (Z, H, Tq), sm)
        extra = {}
        if br == SLIDING:
            extra["window"] = int(kw["WINDOW_SIZE"])
        elif br == COMPRESSION:
            extra["block_ends"] = Blk.reshape(-1)[:Tkv]
        else:
            n = int(kw["N_BLOCKS"])
            extra["indices"] = _view(Blk, (Z, G, Tq, n), sb)
            extra["lprime"] = int(kw["BLOCK_SIZE_SELECTION"])
            extra["causal"] = bool(kw.get("IS_CAUSAL", True))
        if not bwd:
            _ops.attn_fwd(br, q, k, v, float(scale), out=o, L=Lv, M=Mv, **extra)
            return None
        do = _view(dOut, (Z, H, Tq, dv), so)  # dOut shares Out's strides in the reference
        dq = _view(dQ, (Z, H, Tq, dk), sdq)
        dkv = _view(dK, (Z, G, Tkv, dk), sdk)
        dvv = _view(dV, (Z, G, Tkv, dv), sdv)
        _ops.attn_bwd(br, q, k, v, o, do, Lv, Mv, float(scale), dq=dq, dk=dkv, dv=dvv, **extra)
        return None


_nsa_sliding_window_fwd_kernel = _HipKernel("_nsa_sliding_window_fwd_kernel", SLIDING, False)
_nsa_sliding_window_bwd_kernel = _HipKernel("_nsa_sliding_window_bwd_kernel", SLIDING, True)
_nsa_compression_fwd_kernel = _HipKernel("_nsa_compression_fwd_kernel", COMPRESSION, False)
_nsa_compression_bwd_kernel = _HipKernel("_nsa_compression_bwd_kernel", COMPRESSION, True)
_nsa_sparse_selection_fwd_kernel = _HipKernel("_nsa_sparse_selection_fwd_kernel", SELECTION, False)
_nsa_sparse_selection_bwd_kernel = _HipKernel("_nsa_sparse_selection_bwd_kernel", SELECTION, True)


# ==================================================================== autograd wrappers
def _kt(k):
    """[B,G,dk,T] -> the (b, g, time, dk) view."""
    return k.transpose(-1, -2)


def _leaf_grads(q, k, v):
    """dK / dV destinations in the layouts of k ([B,G,dk,T]) and v, overwritten by the
    backward (the kernels take any dK / dV strides): the gradients reach the leaves
    without a layout copy."""
    return dict(dk=_kt(torch.empty_like(k)), dv=torch.empty_like(v), dkdv_overwrite=True)


class CompressionAttention(torch.autograd.Function):
    """Compression branch (reference nsa/kernels.py:34-171).  k_compressed
    [B,G,dk,N], v_compressed [B,G,N,dv], block_ends [N]."""

    @staticmethod
    def forward(ctx, q, k_compressed, v_compressed, block_ends, scale, config):
        o, L, M = _ops.attn_fwd(COMPRESSION, q, _kt(k_compressed), v_compressed, scale, block_ends=block_ends)
        ctx.save_for_backward(q, k_compressed, v_compressed, block_ends, o, L, M)
        ctx.scale = scale
        return o

    @staticmethod
    def backward(ctx, do):
        q, kc, vc, be, o, L, M = ctx.saved_tensors
        dq, dk, dv = _ops.attn_bwd(COMPRESSION, q, _kt(kc), vc, o, do, L, M, ctx.scale, block_ends=be,
                                   **_leaf_grads(q, kc, vc))
        return dq, dk.transpose(-1, -2), dv, None, None, None


class SelectionAttention(torch.autograd.Function):
    """Selection branch (reference nsa/kernels.py:174-365).  indices [B,G,T,n]
    (int32 or int64, -1 = empty); a row with no valid index falls back to block t//l'."""

    @staticmethod
    def forward(ctx, q, k, v, indices, scale, config):
        lp = config.l_prime
        o, L, M = _ops.attn_fwd(SELECTION, q, _kt(k), v, scale, indices=indices, lprime=lp, fallback=True)
        ctx.save_for_backward(q, k, v, indices, o, L, M)
        ctx.scale = scale
        ctx.lprime = lp
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, idx, o, L, M = ctx.saved_tensors
        dq, dk, dv = _ops.attn_bwd(SELECTION, q, _kt(k), v, o, do, L, M, ctx.scale, indices=idx, lprime=ctx.lprime,
                                   fallback=True, **_leaf_grads(q, k, v))
        return dq, dk.transpose(-1, -2), dv, None, None, None


class SlidingWindowAttention(torch.autograd.Function):
    """Sliding-window branch (reference nsa/kernels.py:368-513)."""

    @staticmethod
    def forward(ctx, q, k, v, scale, window_size, config):
        o, L, M = _ops.attn_fwd(SLIDING, q, _kt(k), v, scale, window=window_size)
        ctx.save_for_backward(q, k, v, o, L, M)
        ctx.scale = scale
        ctx.window = window_size
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, L, M = ctx.saved_tensors
        dq, dk, dv = _ops.attn_bwd(SLIDING, q, _kt(k), v, o, do, L, M, ctx.scale, window=ctx.window,
                                   **_leaf_grads(q, k, v))
        return dq, dk.transpose(-1, -2), dv, None, None, None


class NSACore(torch.autograd.Function):
    """The attention core of NSAAttention over one query tensor: the three branches
    (CompressionAttention, SelectionAttention and SlidingWindowAttention, with their
    arguments and layouts), the gate activation of config.gate_mode (sigmoid, or softmax
    over the three gates) applied to gate_logits [B,H,T,3], and the gated mix (GatedMix,
    reference nsa/kernels.py:2429-2463), as one function returning the mixed output.

    The mix is fused into the branch kernels: the sliding-window forward runs last and
    its epilogue writes g0 o_cmp + g1 o_sel + g2 o_win; the branch backwards take the mix's
    output gradient dout unscaled with their gate as a per-row factor (the branch's
    output gradient is g_k dout: dQ is scaled by g_k, the dK / dV probabilities by the
    row's g_k) and write sum_d dout . o_k per row, from which the gate-logit gradient
    follows.  No per-branch output gradient is materialised, and the second and third
    dQ are added into the first's (the dQ kernels' accumulate mode).  Head widths
    without a compiled kernel, or fused_mix = False, take the separate GatedMix passes."""

    fused_mix = True

    @staticmethod
    def forward(ctx, q, k_compressed, v_compressed, block_ends, k_sel, v_sel, indices, k_win, v_win, gate_logits,
                scale, config):
        _ops._check_device(q, gate_logits)
        lp = config.l_prime
        act = GATE_ACT[config.gate_mode]
        cdt = _ops.compute_dtype(q.dtype)
        B, H, T, dk = q.shape
        dv = v_compressed.shape[-1]
        fused = NSACore.fused_mix and _ops.kernel_dims(dk, dv) == (dk, dv)
        ctx.scale, ctx.lprime, ctx.window, ctx.gdtype, ctx.act, ctx.fused = (scale, lp, config.w, gate_logits.dtype,
                                                                             act, fused)
        if fused:
            # branch outputs and the mix in [B,T,H,dv] storage (the module's layout)
            def bthd():
                return torch.empty(B, T, H, dv, device=q.device, dtype=cdt).permute(0, 2, 1, 3)

            o_c, o_s, o_w, out = bthd(), bthd(), bthd(), bthd()
            gates = _gate_activation(gate_logits, act)  # [3,B,H,T] fp32
            _, Lc, Mc = _ops.attn_fwd(COMPRESSION, q, _kt(k_compressed), v_compressed, scale, block_ends=block_ends,
                                      out=o_c)
            _, Ls, Ms = _ops.attn_fwd(SELECTION, q, _kt(k_sel), v_sel, scale, indices=indices, lprime=lp,
                                      fallback=True, out=o_s)
            _, Lw, Mw = _ops.attn_fwd(SLIDING, q, _kt(k_win), v_win, scale, window=config.w, out=o_w,
                                      mix=(o_c, o_s, gates, out))
            ctx.save_for_backward(q, k_compressed, v_compressed, block_ends, k_sel, v_sel, indices, k_win, v_win,
                                  gates, o_c, o_s, o_w, Lc, Mc, Ls, Ms, Lw, Mw)
            return out.to(q.dtype)
        o_c, Lc, Mc = _ops.attn_fwd(COMPRESSION, q, _kt(k_compressed), v_compressed, scale, block_ends=block_ends)
        o_s, Ls, Ms = _ops.attn_fwd(SELECTION, q, _kt(k_sel), v_sel, scale, indices=indices, lprime=lp,
                                    fallback=True)
        o_w, Lw, Mw = _ops.attn_fwd(SLIDING, q, _kt(k_win), v_win, scale, window=config.w)
        os_ = [t.to(cdt).contiguous() for t in (o_c, o_s, o_w)]
        g = gate_logits.to(cdt)
        out = _mix_fwd(os_, g, act)
        ctx.save_for_backward(q, k_compressed, v_compressed, block_ends, k_sel, v_sel, indices, k_win, v_win, g,
                              *os_, Lc, Mc, Ls, Ms, Lw, Mw)
        return out.to(q.dtype)

    @staticmethod
    def backward(ctx, dout):
        (q, kc, vc, be, ks, vs, idx, kw, vw, g, o_c, o_s, o_w, Lc, Mc, Ls, Ms, Lw, Mw) = ctx.saved_tensors
        sc = ctx.scale
        # dQ in q's own layout (no transposing copy on the way back to the projection)
        dq = torch.empty_like(q, dtype=_ops.compute_dtype(q.dtype))
        if ctx.fused:
            d = dout.to(o_c.dtype)
            if d.stride() != o_c.stride():  # one copy into the branch outputs' layout
                d = torch.empty_like(o_c).copy_(d)
            # r_k = sum_d dout . o_k for the three branches in one pass (dout read once): the
            # gate gradient's inputs and each branch's row sums, so no branch reads o_k again
            rdot = torch.empty(g.shape, device=q.device, dtype=torch.float32)  # [3,B,H,T]
            B, H, T = q.shape[:3]
            _lib.call("nsa_mix_row_dots", _ops._ptr(d), _ops._ptr(o_c), _ops._ptr(o_s), _ops._ptr(o_w),
                      *o_c.stride()[:3], _ops._ptr(rdot), B, H, T, o_c.shape[-1], _ops._dtype_code(d.dtype),
                      _ops._stream(q.device))
            # dK / dV written straight into buffers with the inputs' own strides (the
            # kernels take any dK / dV strides): the gradients need no layout copy on the
            # way back to the projections
            cdt = _ops.compute_dtype(q.dtype)

            def like(t):
                return torch.empty_like(t, dtype=cdt)

            dkc, dvc, dks, dvs, dkw, dvw = like(_kt(kc)), like(vc), like(_kt(ks)), like(vs), like(_kt(kw)), like(vw)
            if (_ops.dq_deferrable(COMPRESSION, q, _kt(kc), vc) and _ops.dq_deferrable(SLIDING, q, _kt(kw), vw,
                                                                                          window=ctx.window)):
                # both dense branches store dS: the selection dQ is written first, and the
                # sliding-window dQ pass adds the compression dQ as well, so the running dQ
                # is read and written once for the two
                _ops.attn_bwd(SELECTION, q, _kt(ks), vs, o_s, d, Ls, Ms, sc, indices=idx, lprime=ctx.lprime,
                              fallback=True, dq=dq, dk=dks, dv=dvs, dkdv_overwrite=True, row_gate=g[1],
                              delta=rdot[1])
                pend = _ops.DeferredDq()
                _ops.attn_bwd(COMPRESSION, q, _kt(kc), vc, o_c, d, Lc, Mc, sc, block_ends=be, dq=dq, dk=dkc,
                              dv=dvc, dkdv_overwrite=True, row_gate=g[0], delta=rdot[0], defer_dq=pend)
                _ops.attn_bwd(SLIDING, q, _kt(kw), vw, o_w, d, Lw, Mw, sc, window=ctx.window, dq=dq,
                              dq_accumulate=True, dk=dkw, dv=dvw, dkdv_overwrite=True, row_gate=g[2], delta=rdot[2],
                              pair=pend)
            else:
                _ops.attn_bwd(COMPRESSION, q, _kt(kc), vc, o_c, d, Lc, Mc, sc, block_ends=be, dq=dq, dk=dkc, dv=dvc,
                              dkdv_overwrite=True, row_gate=g[0], delta=rdot[0])
                _ops.attn_bwd(SELECTION, q, _kt(ks), vs, o_s, d, Ls, Ms, sc, indices=idx, lprime=ctx.lprime,
                              fallback=True, dq=dq, dq_accumulate=True, dk=dks, dv=dvs, dkdv_overwrite=True,
                              row_gate=g[1], delta=rdot[1])
                _ops.attn_bwd(SLIDING, q, _kt(kw), vw, o_w, d, Lw, Mw, sc, window=ctx.window, dq=dq,
                              dq_accumulate=True, dk=dkw, dv=dvw, dkdv_overwrite=True, row_gate=g[2], delta=rdot[2])
            dg = _gate_activation_grad(g, rdot, ctx.act, ctx.gdtype)
        else:
            dos, dg, deltas = _mix_bwd(dout, [o_c, o_s, o_w], g, want_delta=True, act=ctx.act)
            _, dkc, dvc = _ops.attn_bwd(COMPRESSION, q, _kt(kc), vc, o_c, dos[0], Lc, Mc, sc, block_ends=be, dq=dq,
                                        delta=deltas[0])
            _, dks, dvs = _ops.attn_bwd(SELECTION, q, _kt(ks), vs, o_s, dos[1], Ls, Ms, sc, indices=idx,
                                        lprime=ctx.lprime, fallback=True, dq=dq, dq_accumulate=True, delta=deltas[1])
            _, dkw, dvw = _ops.attn_bwd(SLIDING, q, _kt(kw), vw, o_w, dos[2], Lw, Mw, sc, window=ctx.window, dq=dq,
                                        dq_accumulate=True, delta=deltas[2])
        return (dq.to(q.dtype), dkc.transpose(-1, -2), dvc, None, dks.transpose(-1, -2), dvs, None,
                dkw.transpose(-1, -2), dvw, dg if dg.dtype == ctx.gdtype else dg.to(ctx.gdtype), None, None)


@functools.lru_cache(maxsize=32)
def _block_ends(n_pad: int, n_act: int, d: int, l: int, device) -> torch.Tensor:
    """block_ends [n_pad] int32: block i ends at token i*d + l - 1 for i < n_act, the
    padding blocks at 999999 (never visible).  Built once per shape and device: the
    per-step rebuild was five small launches.  Built outside inference mode, so a tensor
    first made by an eval step under torch.inference_mode() can still be saved for a
    later training step's backward.  Shared: only module-internal callers get it
    (NSAAttention.compress_tokens hands out a copy)."""
    with torch.inference_mode(False):
        be = torch.full((n_pad,), 999999, device=device, dtype=torch.int32)
        if n_act > 0:
            be[:n_act] = torch.arange(n_act, device=device, dtype=torch.int32) * d + (l - 1)
    return be


def _gate_activation(z, act):
    """Gates [3,B,H,T] fp32 from the gate input z [B,H,T,3] (any strides): z itself,
    sigmoid(z) or softmax over the three (reference nsa/kernels.py:2436-2440), one HIP
    pass (nsa_gate_act_fwd)."""
    B, H, T, _ = z.shape
    if z.dtype not in (torch.float32, torch.bfloat16):
        z = z.float()
    g = torch.empty(3, B, H, T, device=z.device, dtype=torch.float32)
    _lib.call("nsa_gate_act_fwd", _ops._ptr(z), *z.stride(), _ops._ptr(g), B, H, T, act, _ops._dtype_code(z.dtype),
              _ops._stream(z.device))
    return g


def _gate_activation_grad(a, r, act, dtype):
    """Gradient [B,H,T,3] of the gate input from the gates a and r_k = sum_d dout . o_k
    (both [3,B,H,T] fp32): r (identity), r a (1 - a) (sigmoid), a (r - sum_j a_j r_j)
    (softmax); one HIP pass (nsa_gate_act_bwd), in dtype when fp32 / bf16, else fp32."""
    _, B, H, T = a.shape
    dt = dtype if dtype in (torch.float32, torch.bfloat16) else torch.float32
    dz = torch.empty(B, H, T, 3, device=a.device, dtype=dt)
    _lib.call("nsa_gate_act_bwd", _ops._ptr(a), _ops._ptr(r), _ops._ptr(dz), *dz.stride(), B, H, T, act,
              _ops._dtype_code(dt), _ops._stream(a.device))
    return dz


def _wgrad_hip(dy2, x2, W) -> bool:
    """Whether nsa_wgrad computes dW = dy2^T x2 here: bf16 on the GPU, rows with unit
    feature stride and 16-byte aligned, both widths multiples of 64 (rows that overlap,
    e.g. a gradient broadcast along the rows, take the batched GEMM)."""
    return (dy2.is_cuda and dy2.dtype == x2.dtype == W.dtype == torch.bfloat16
            and W.shape[0] % 64 == 0 and W.shape[1] % 64 == 0 and dy2.stride(-1) == 1 and x2.stride(-1) == 1
            and dy2.stride(0) % 8 == 0 and x2.stride(0) % 8 == 0 and dy2.data_ptr() % 16 == 0
            and x2.data_ptr() % 16 == 0
            and dy2.stride(0) >= W.shape[0] and x2.stride(0) >= W.shape[1])


class _LinearSplitK(torch.autograd.Function):
    """y = x W^T (+ b) whose weight gradient is a reduction over every row of x (all
    B*G*T tokens for the compression MLP, against a 384 x 192 output): a single GEMM of
    that shape has too few output tiles to fill the GPU.  bf16 takes the HIP split-row
    reduction (nsa_wgrad: fixed row chunks on the matrix cores, fp32 partial tiles added
    in order); otherwise S row chunks go through one batched GEMM with fp32 partials,
    then summed."""

    @staticmethod
    def forward(ctx, x, W, b):
        ctx.save_for_backward(x, W)
        ctx.has_b = b is not None
        return F.linear(x, W, b)

    @staticmethod
    def backward(ctx, dy):
        x, W = ctx.saved_tensors
        dx = dW = db = None
        if ctx.needs_input_grad[0]:
            dx = dy @ W
        dy2 = dy.reshape(-1, dy.shape[-1])
        if ctx.needs_input_grad[1]:
            x2 = x.reshape(-1, x.shape[-1])
            rows = x2.shape[0]
            if _wgrad_hip(dy2, x2, W):
                dW = torch.empty(W.shape, device=W.device, dtype=W.dtype)
                ws = torch.empty(max(_lib.size("nsa_wgrad_workspace_size", rows, W.shape[0], W.shape[1]), 1),
                                 device=W.device, dtype=torch.uint8)
                _lib.call("nsa_wgrad", _ops._ptr(dy2), dy2.stride(0), _ops._ptr(x2), x2.stride(0), rows, W.shape[0],
                          W.shape[1], _ops._ptr(dW), dW.stride(0), _lib.NSA_BF16, _ops._ptr(ws), ws.numel(),
                          _ops._stream(W.device))
            else:
                S = 64
                while S > 1 and (rows % S or rows // S < 256):
                    S //= 2
                if S > 1 and dy2.is_cuda:
                    part = torch.bmm(dy2.view(S, rows // S, -1).transpose(1, 2), x2.view(S, rows // S, -1),
                                     out_dtype=torch.float32)
                    dW = part.sum(0).to(W.dtype)
                else:
                    dW = dy2.t() @ x2
        if ctx.has_b and ctx.needs_input_grad[2]:
            db = dy2.sum(0)
        return dx, dW, db


class _SplitCols(torch.autograd.Function):
    """(W[:, :k], W[:, k:]) whose backward writes W's gradient as one concatenation of
    the two parts' gradients (two slicing backwards would zero-fill and copy each part
    into its own full-size gradient, then add the two)."""

    @staticmethod
    def forward(ctx, W, k):
        ctx.k, ctx.n = k, W.shape[1]
        return W[:, :k], W[:, k:]

    @staticmethod
    def backward(ctx, g1, g2):
        if g1 is None and g2 is None:
            return None, None
        ref = g1 if g1 is not None else g2
        if g1 is None:
            g1 = ref.new_zeros(ref.shape[0], ctx.k)
        if g2 is None:
            g2 = ref.new_zeros(ref.shape[0], ctx.n - ctx.k)
        return torch.cat([g1, g2], dim=1), None


class _CompressPool(torch.autograd.Function):
    """R[i] = mean_u relu(Y[d*i+u] + C[u]),  V_cmp[i] = mean_u v[d*i+u]  (HIP)."""

    @staticmethod
    def forward(ctx, Y, C, v, l, d, n_act, token_major=False):
        """Y, v: [B,G,T,*], or [B,T,G,*] with token_major (the storage order of the
        module's projections: no transposing copy)."""
        cdt = _ops.compute_dtype(Y.dtype)
        Yc, Cc, vc = Y.to(cdt).contiguous(), C.to(cdt).contiguous(), v.to(cdt).contiguous()
        if token_major:
            B, T, G, W = Yc.shape
        else:
            B, G, T, W = Yc.shape
        dv = vc.shape[-1]
        R = torch.empty(B, G, n_act, W, device=Y.device, dtype=cdt)
        Vc = torch.empty(B, G, n_act, dv, device=Y.device, dtype=cdt)
        _lib.call("nsa_compress_pool_fwd", _ops._ptr(Yc), _ops._ptr(Cc), _ops._ptr(vc), _ops._ptr(R), _ops._ptr(Vc),
                  B, G, T, W, dv, l, d, n_act, int(bool(token_major)), _ops._dtype_code(cdt), _ops._stream(Y.device))
        ctx.save_for_backward(Yc, Cc)
        ctx.meta = (l, d, n_act, dv, Y.dtype, C.dtype, v.dtype, bool(token_major), (B, G, T, W))
        return R.to(Y.dtype), Vc.to(v.dtype)

    @staticmethod
    def backward(ctx, dR, dVc):
        Yc, Cc = ctx.saved_tensors
        l, d, n_act, dv, ydt, cdt_in, vdt, tm, (B, G, T, W) = ctx.meta
        cdt = Yc.dtype
        dRc = (dR if dR is not None else torch.zeros(B, G, n_act, W, device=Yc.device)).to(cdt).contiguous()
        dVcc = (dVc if dVc is not None else torch.zeros(B, G, n_act, dv, device=Yc.device)).to(cdt).contiguous()
        dY = torch.empty_like(Yc)
        dV = torch.empty(*((B, T, G) if tm else (B, G, T)), dv, device=Yc.device, dtype=cdt)
        dC = torch.empty(l, W, device=Yc.device, dtype=torch.float32)
        _lib.call("nsa_compress_pool_bwd", _ops._ptr(Yc), _ops._ptr(Cc), _ops._ptr(dRc), _ops._ptr(dVcc),
                  _ops._ptr(dY), _ops._ptr(dC), _ops._ptr(dV), B, G, T, W, dv, l, d, n_act, int(tm),
                  _ops._dtype_code(cdt), _ops._stream(Yc.device))
        return dY.to(ydt), dC.to(cdt_in), dV.to(vdt), None, None, None, None


# ============================================================== selection (Eq. 9 / 10)
GATE_ACT = {"none": 0, "sigmoid": 1, "softmax": 2}  # gate_act codes of nsa_gate_mix_*


def _mix_fwd(os_, g, act=0):
    """out = sum_k a(g)[..., k] o_k over compute-dtype contiguous branch outputs [B,H,T,dv]
    (a = identity, sigmoid or softmax over the 3 gates: act 0, 1, 2); the result is a
    [B,H,T,dv] view of [B,T,H,dv] storage."""
    B, H, T, dv = os_[0].shape
    cdt = os_[0].dtype
    out = torch.empty(B, T, H, dv, device=os_[0].device, dtype=cdt).permute(0, 2, 1, 3)
    so, sg, sx = os_[0].stride(), g.stride(), out.stride()
    _lib.call("nsa_gate_mix_fwd", *[_ops._ptr(t) for t in os_], so[0], so[1], so[2], _ops._ptr(g), *sg,
              _ops._ptr(out), sx[0], sx[1], sx[2], B, H, T, dv, act, _ops._dtype_code(cdt),
              _ops._stream(out.device))
    return out


def _mix_bwd(dout, os_, g, want_delta=False, act=0):
    """With gates a = act(g): (d o_k = a[..., k] dout for k < 3, the fp32 gradient [B,H,T,3]
    of g (from sum_d dout o_k through the activation), and with want_delta the row sums
    delta [3,B,H,T] fp32, delta[k] = a[..., k] sum_d dout o_k)."""
    cdt = os_[0].dtype
    B, H, T, dv = os_[0].shape
    d = dout.to(cdt)
    if d.stride(-1) != 1 or (d.stride(2) * d.element_size()) % 16 or (d.stride(1) * d.element_size()) % 16:
        d = d.contiguous()
    dos = [torch.empty(B, H, T, dv, device=d.device, dtype=cdt) for _ in range(3)]
    dg = torch.empty(B, H, T, 3, device=d.device, dtype=torch.float32)
    delta = torch.empty(3, B, H, T, device=d.device, dtype=torch.float32) if want_delta else None
    sd, so, sg = d.stride(), os_[0].stride(), g.stride()
    _lib.call("nsa_gate_mix_bwd", _ops._ptr(d), sd[0], sd[1], sd[2], *[_ops._ptr(t) for t in os_], so[0], so[1],
              so[2], _ops._ptr(g), *sg, *[_ops._ptr(t) for t in dos], _ops._ptr(dg), _ops._ptr(delta), B, H, T, dv,
              act, _ops._dtype_code(cdt), _ops._stream(d.device))
    return (dos, dg, delta) if want_delta else (dos, dg)


class GatedMix(torch.autograd.Function):
    """o = o_cmp * g[..., 0] + o_sel * g[..., 1] + o_win * g[..., 2] (NSAAttention.forward,
    reference nsa/kernels.py:2446-2463) as one fused HIP pass each way.  Branch outputs
    [B,H,T,dv], gates [B,H,T,3]; the result is a [B,H,T,dv] view of [B,T,H,dv] storage,
    so the module's transpose + reshape to [B,T,H*dv] copies nothing."""

    @staticmethod
    def forward(ctx, o_cmp, o_sel, o_win, gates):
        _ops._check_device(o_cmp, o_sel, o_win, gates)
        cdt = _ops.compute_dtype(o_cmp.dtype)
        os_ = [t.to(cdt).contiguous() for t in (o_cmp, o_sel, o_win)]
        g = gates.to(cdt)
        out = _mix_fwd(os_, g)
        ctx.save_for_backward(*os_, g)
        ctx.dtypes = (o_cmp.dtype, o_sel.dtype, o_win.dtype, gates.dtype)
        return out.to(o_cmp.dtype)

    @staticmethod
    def backward(ctx, dout):
        o_c, o_s, o_w, g = ctx.saved_tensors
        dos, dg = _mix_bwd(dout, [o_c, o_s, o_w], g)
        dts = ctx.dtypes
        return dos[0].to(dts[0]), dos[1].to(dts[1]), dos[2].to(dts[2]), dg.to(dts[3])


def derive_selection_from_compression_per_timestep(compression_scores: torch.Tensor,
                                                   config: NSAConfig) -> torch.Tensor:
    """Eq. 9 (reference nsa/kernels.py:1920-1962): p_slc[j] = sum_{m<l'/d} sum_{n<l/d}
    p_cmp[s*j+m+n], accumulated in the same (m, n) order, vectorised over j."""
    B, H, T, nc = compression_scores.shape
    assert config.l % config.d == 0 and config.l_prime % config.d == 0
    a = config.l // config.d
    s = config.l_prime // config.d
    nsel = (nc + s - 1) // s
    padded = F.pad(compression_scores, (0, nsel * s + s + a - nc))
    out = torch.zeros(B, H, T, nsel, device=compression_scores.device, dtype=compression_scores.dtype)
    for m in range(s):
        for n in range(a):
            # p_cmp[s*j + m + n] for all j; entries past nc are the zero padding
            out += padded[..., m + n: m + n + s * nsel: s][..., :nsel]
    return out


def select_top_k_blocks_per_query_with_gqa(selection_scores: torch.Tensor, config: NSAConfig,
                                           always_include_blocks: Optional[List[int]] = None) -> torch.Tensor:
    """Eq. 10 + top-n (reference nsa/kernels.py:1965-2040): head-sum per KV group,
    stable descending sort (ties -> lower block index), fixed blocks
    [0, max(0,(t-l')//l'), t//l'] merged in front and de-duplicated in order, -1
    padding.  Vectorised: no per-row host loop."""
    B, H, T, nb = selection_scores.shape
    G = config.n_kv_groups
    agg = selection_scores.view(B, G, config.heads_per_group, T, nb).sum(dim=2)
    k = min(config.n, nb)
    _, order = torch.sort(agg, dim=-1, descending=True, stable=True)
    top = order[..., :k]
    dev = selection_scores.device
    if config.include_fixed_in_selection and config.n_fixed > 0:
        pos = torch.arange(T, device=dev)
        fixed = torch.stack([torch.zeros_like(pos), torch.clamp((pos - config.l_prime) // config.l_prime, min=0),
                             pos // config.l_prime], dim=-1)
        cand = torch.cat([fixed.view(1, 1, T, 3).expand(B, G, T, 3), top], dim=-1)  # [B,G,T,3+k]
        c = cand.shape[-1]
        earlier = torch.triu(torch.ones(c, c, dtype=torch.bool, device=dev), diagonal=1)  # [i, j]: i < j
        dup = ((cand.unsqueeze(-1) == cand.unsqueeze(-2)) & earlier).any(dim=-2)  # seen at an earlier slot
        keep = ~dup
        rank = torch.cumsum(keep.to(torch.int64), dim=-1) - 1
        out = torch.full((B, G, T, config.n + 1), -1, device=dev, dtype=torch.long)
        slot = torch.where(keep & (rank < config.n), rank, torch.full_like(rank, config.n))
        out.scatter_(-1, slot, torch.where(slot < config.n, cand, torch.full_like(cand, -1)))
        return out[..., :config.n]
    if top.shape[-1] < config.n:
        pad = torch.full((B, G, T, config.n - top.shape[-1]), -1, device=dev, dtype=top.dtype)
        return torch.cat([top, pad], dim=-1)
    return top[..., :config.n]


def score_and_select(q: torch.Tensor, k_compressed: torch.Tensor, block_ends: torch.Tensor, scale: float,
                     config: NSAConfig, return_scores: bool = False, q_offset: int = 0):
    """Fused Eq. 8 -> 9 -> 10 -> top-n on the GPU (one HIP kernel).

    q [B,H,T,dk], k_compressed [B,G,dk,N], block_ends [N] -> indices [B,G,T,n] int64
    (and the fp32 p_cmp [B,H,T,N] / p_slc [B,H,T,nsel] when return_scores).  q_offset:
    absolute position of query row 0 (decode past a cache)."""
    _ops._check_device(q, k_compressed, block_ends)
    B, H, T, dk = q.shape
    G, N = k_compressed.shape[1], k_compressed.shape[-1]
    cdt = _ops.compute_dtype(q.dtype)
    qc = q.to(cdt)
    # the kernel reads each compressed key as one row: [B,G,N,dk] storage
    kc = k_compressed.to(cdt).transpose(-1, -2).contiguous().transpose(-1, -2)
    be = block_ends.to(torch.int32).contiguous()
    s = config.l_prime // config.d
    nsel = (N + s - 1) // s
    out = torch.empty(B, G, T, config.n, device=q.device, dtype=torch.long)
    pc = torch.empty(B, H, T, N, device=q.device, dtype=torch.float32) if return_scores else None
    ps = torch.empty(B, H, T, nsel, device=q.device, dtype=torch.float32) if return_scores else None
    ws_bytes = _lib.load().nsa_score_topn_workspace_size(B, H, G, T, dk, N, config.n)
    ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
    if q_offset < 0:
        raise ValueError("q_offset must be >= 0")
    name, off = ("nsa_score_topn_ex", (int(q_offset),)) if q_offset else ("nsa_score_topn", ())
    _lib.call(name, _ops._ptr(qc), _ops._ptr(kc), _ops._ptr(be), _ops._ptr(out), _ops._ptr(pc),
              _ops._ptr(ps), *qc.stride(), *kc.stride(), *out.stride(), B, H, G, T, dk, N, config.l, config.d,
              config.l_prime, config.n, int(bool(config.include_fixed_in_selection)), int(config.n_fixed),
              _ops._dtype_code(cdt), float(scale), *off, _ops._ptr(ws), ws_bytes, _ops._stream(q.device))
    if return_scores:
        return out, pc, ps
    return out


# ========================================================================= decode state
def _n_pad(n_act: int) -> int:
    n = 1
    while n < n_act:
        n *= 2
    return n


class NSAKVCache:
    """Decode state of one NSAAttention layer (not in the reference, whose module only
    runs whole sequences): the projected keys / values of every past token for the three
    branches ([B,G,max_len,d] each) and the compressed tokens of every completed block
    (K_cmp [B,G,dk,Np], V_cmp [B,G,Np,dv], block_ends [Np], Np a power of two covering
    max_len, unused entries 999999 as compress_tokens pads them).  Filled by
    NSAAttention.prefill and extended one token at a time by NSAAttention.decode."""

    def __init__(self, config: NSAConfig, batch: int, max_len: int, device, dtype):
        c = config
        G, dk, dv = c.n_kv_groups, c.head_dim_qk, c.head_dim_v
        self.config, self.max_len, self.length = config, max_len, 0

        def buf(d):
            return torch.zeros(batch, G, max_len, d, device=device, dtype=dtype)

        self.k_cmp_in, self.v_cmp_in = buf(dk), buf(dv)
        self.k_sel, self.v_sel = buf(dk), buf(dv)
        self.k_win, self.v_win = buf(dk), buf(dv)
        n_max = max((max_len - c.l) // c.d + 1, 0)
        np_max = _n_pad(max(n_max, 1))
        self.K_cmp = torch.zeros(batch, G, dk, np_max, device=device, dtype=dtype)
        self.V_cmp = torch.zeros(batch, G, np_max, dv, device=device, dtype=dtype)
        self.block_ends = torch.full((np_max,), 999999, device=device, dtype=torch.int32)
        self.n_act = 0


# ========================================================================= the module
class NSAAttention(torch.nn.Module):
    """Native Sparse Attention layer (reference nsa/kernels.py:2043-2507): projections,
    compression with MLP pooling, fused Eq. 8-10 selection, the three HIP attention
    branches, gated mixing and the output projection."""

    def __init__(self, config: NSAConfig):
        super().__init__()
        self.config = config
        c = config
        lin = torch.nn.Linear
        self.q_proj = lin(c.d_model, c.n_heads * c.head_dim_qk, bias=c.use_bias)
        self.k_compress = lin(c.d_model, c.n_kv_groups * c.head_dim_qk, bias=c.use_bias)
        self.v_compress = lin(c.d_model, c.n_kv_groups * c.head_dim_v, bias=c.use_bias)
        self.k_select = lin(c.d_model, c.n_kv_groups * c.head_dim_qk, bias=c.use_bias)
        self.v_select = lin(c.d_model, c.n_kv_groups * c.head_dim_v, bias=c.use_bias)
        self.k_sliding = lin(c.d_model, c.n_kv_groups * c.head_dim_qk, bias=c.use_bias)
        self.v_sliding = lin(c.d_model, c.n_kv_groups * c.head_dim_v, bias=c.use_bias)
        self.pos_embed = torch.nn.Embedding(c.l, c.l)
        self.compress_mlp = torch.nn.Sequential(
            lin(c.head_dim_qk + c.l, c.head_dim_qk * 2), torch.nn.ReLU(), lin(c.head_dim_qk * 2, c.head_dim_qk))
        self.gate_mlp = torch.nn.Sequential(
            lin(c.d_model, c.d_model // 2), torch.nn.ReLU(), lin(c.d_model // 2, 3 * c.n_heads))
        self.o_proj = lin(c.n_heads * c.head_dim_v, c.d_model, bias=c.use_bias)
        self.dropout = torch.nn.Dropout(c.dropout_p)
        self.scale = 1.0 / math.sqrt(c.head_dim_qk)

    def compress_tokens(self, keys: torch.Tensor, values: torch.Tensor
                        ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, int]:
        """keys [B,G,T,dk], values [B,G,T,dv] -> (K_cmp [B,G,dk,Np], V_cmp [B,G,Np,dv],
        block_ends [Np] int32, n_actual) with Np the power-of-two padded block count
        (padding: zero keys/values, block_ends 999999), as nsa/kernels.py:2119-2208.
        block_ends is the caller's own tensor (a copy of the module's cached one)."""
        kc, vc, be, n_act = self._compress_tokens(keys, values)
        return kc, vc, be.clone(), n_act

    def _compress_tokens(self, keys: torch.Tensor, values: torch.Tensor):
        """compress_tokens with block_ends the shared cached tensor (module-internal: it
        is never modified)."""
        c = self.config
        B, G, T, dk = keys.shape
        dv = values.shape[-1]
        n_act = (T - c.l) // c.d + 1
        n_pad = 1
        while n_pad < n_act:
            n_pad *= 2
        dev, dt = keys.device, keys.dtype
        block_ends = _block_ends(n_pad, n_act, c.d, c.l, dev)
        if n_act <= 0:
            return (torch.zeros(B, G, dk, n_pad, device=dev, dtype=dt), torch.zeros(B, G, n_pad, dv, device=dev, dtype=dt),
                    block_ends, n_act)
        l1, l2 = self.compress_mlp[0], self.compress_mlp[2]
        W1k, W1p = _SplitCols.apply(l1.weight, dk)
        # keys / values as the module's projections store them ([B,T,G,d], viewed
        # [B,G,T,d]) are used in that order: the GEMM and the pooling then read them
        # without a transposing copy, and their gradients come back in the same layout
        tm = G > 1 and keys.transpose(1, 2).is_contiguous() and values.transpose(1, 2).is_contiguous()
        kin = keys.transpose(1, 2) if tm else keys
        Y = _LinearSplitK.apply(kin, W1k.to(dt), None)                           # [B,G,T,2dk] ([B,T,G,2dk])
        C = F.linear(self.pos_embed.weight.to(dt), W1p.to(dt),
                     l1.bias.to(dt) if l1.bias is not None else None)             # [l,2dk]
        R, Vc = _CompressPool.apply(Y, C, values.transpose(1, 2) if tm else values, c.l, c.d, n_act, tm)
        Kc = _LinearSplitK.apply(R, l2.weight.to(dt), l2.bias.to(dt) if l2.bias is not None else None)  # [B,G,n,dk]
        Kc = F.pad(Kc, (0, 0, 0, n_pad - n_act)).transpose(-1, -2)               # [B,G,dk,Np]
        Vc = F.pad(Vc, (0, 0, 0, n_pad - n_act))                                 # [B,G,Np,dv]
        return Kc, Vc, block_ends, n_act

    # ------------------------------------------------------------------ decode
    def _project_kv(self, x: torch.Tensor):
        c = self.config
        B, T, _ = x.shape
        G, dk, dv = c.n_kv_groups, c.head_dim_qk, c.head_dim_v

        def heads(proj, width):
            return proj(x).view(B, T, G, width).transpose(1, 2)

        return (heads(self.k_compress, dk), heads(self.v_compress, dv), heads(self.k_select, dk),
                heads(self.v_select, dv), heads(self.k_sliding, dk), heads(self.v_sliding, dv))

    def _add_blocks(self, cache: NSAKVCache) -> None:
        """Compress every block the cache's tokens complete (block i covers tokens
        i*d .. i*d+l-1): one compress_tokens call over the tokens of all new blocks."""
        c = self.config
        n_new = (cache.length - c.l) // c.d + 1 if cache.length >= c.l else 0
        i0 = cache.n_act
        if n_new <= i0:
            return
        lo, hi = i0 * c.d, (n_new - 1) * c.d + c.l
        kc, vc, _, n1 = self._compress_tokens(cache.k_cmp_in[:, :, lo:hi], cache.v_cmp_in[:, :, lo:hi])
        assert n1 == n_new - i0
        cache.K_cmp[..., i0:n_new] = kc[..., :n1]
        cache.V_cmp[:, :, i0:n_new] = vc[:, :, :n1]
        cache.block_ends[i0:n_new] = torch.arange(i0, n_new, device=cache.block_ends.device,
                                                  dtype=torch.int32) * c.d + (c.l - 1)
        cache.n_act = n_new

    @torch.no_grad()
    def prefill(self, hidden_states: torch.Tensor, cache: NSAKVCache) -> None:
        """Append the projected keys / values of hidden_states [B,T,D] to the cache and
        compress the blocks they complete (no attention output: run forward for that)."""
        B, T, _ = hidden_states.shape
        t0 = cache.length
        if t0 + T > cache.max_len:
            raise ValueError(f"cache holds {cache.max_len} tokens, {t0 + T} requested")
        bufs = (cache.k_cmp_in, cache.v_cmp_in, cache.k_sel, cache.v_sel, cache.k_win, cache.v_win)
        for dst, src in zip(bufs, self._project_kv(hidden_states)):
            dst[:, :, t0:t0 + T] = src.to(dst.dtype)
        cache.length = t0 + T
        self._add_blocks(cache)

    @torch.no_grad()
    def decode(self, hidden_states: torch.Tensor, cache: NSAKVCache, output_attentions: bool = False):
        """One decode step (not in the reference): hidden_states [B,1,D] is the token at
        position t = cache.length.  Its keys / values join the cache, then the three
        branches, the gates and the mix run for its query alone at absolute position t,
        through the HIP kernels' decode extensions (scoring, attention forward with
        q_offset = t).  Returns (out [B,1,D], info) as forward does for that row."""
        c = self.config
        B, T, D = hidden_states.shape
        if T != 1:
            raise ValueError("decode takes one token per step")
        H, dk, dv = c.n_heads, c.head_dim_qk, c.head_dim_v
        t = cache.length
        self.prefill(hidden_states, cache)
        x = hidden_states
        q = self.q_proj(x).view(B, 1, H, dk).transpose(1, 2).contiguous()           # [B,H,1,dk]
        n_pad = _n_pad(max(cache.n_act, 1)) if cache.n_act > 0 else 1
        kc = cache.K_cmp[..., :n_pad]
        vc = cache.V_cmp[:, :, :n_pad]
        be = cache.block_ends[:n_pad]
        sel = score_and_select(q, kc, be, self.scale, c, return_scores=output_attentions, q_offset=t)
        indices = sel[0] if output_attentions else sel
        n = t + 1
        o_c, _, _ = _ops.attn_fwd(COMPRESSION, q, _kt(kc), vc, self.scale, block_ends=be, q_offset=t)
        o_s, _, _ = _ops.attn_fwd(SELECTION, q, cache.k_sel[:, :, :n], cache.v_sel[:, :, :n], self.scale,
                                  indices=indices, lprime=c.l_prime, fallback=True, q_offset=t)
        o_w, _, _ = _ops.attn_fwd(SLIDING, q, cache.k_win[:, :, :n], cache.v_win[:, :, :n], self.scale, window=c.w,
                                  q_offset=t)
        gate_logits = self.gate_mlp(x).view(B, 1, H, 3).permute(0, 2, 1, 3)
        cdt = _ops.compute_dtype(q.dtype)
        os_ = [o.to(cdt).contiguous() for o in (o_c, o_s, o_w)]
        o = _mix_fwd(os_, gate_logits.to(cdt), GATE_ACT[c.gate_mode]).to(q.dtype)
        out = self.dropout(self.o_proj(o.transpose(1, 2).reshape(B, 1, H * dv)))  # as forward does
        info = None
        if output_attentions:
            gates = torch.softmax(gate_logits, dim=-1) if c.gate_mode == "softmax" else torch.sigmoid(gate_logits)
            info = {"compression_scores": sel[1], "selection_scores": sel[2], "selected_indices": indices,
                    "gates": gates.permute(0, 2, 1, 3)}
        return out, info

    def forward(self, hidden_states: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                output_attentions: bool = False) -> Tuple[torch.Tensor, Optional[Dict]]:
        c = self.config
        B, T, D = hidden_states.shape
        H, G, dk, dv = c.n_heads, c.n_kv_groups, c.head_dim_qk, c.head_dim_v
        x = hidden_states

        def heads(proj, n, width):
            return proj(x).view(B, T, n, width).transpose(1, 2)

        q = heads(self.q_proj, H, dk)
        k_comp, v_comp = heads(self.k_compress, G, dk), heads(self.v_compress, G, dv)
        k_sel, v_sel = heads(self.k_select, G, dk), heads(self.v_select, G, dv)
        k_win, v_win = heads(self.k_sliding, G, dk), heads(self.v_sliding, G, dv)

        k_cmp, v_cmp, block_ends, _ = self._compress_tokens(k_comp, v_comp)
        with torch.no_grad():
            sel = score_and_select(q.detach(), k_cmp.detach(), block_ends, self.scale, c, return_scores=output_attentions)
        if output_attentions:
            indices, p_cmp, p_slc = sel
        else:
            indices, p_cmp, p_slc = sel, None, None

        gate_logits = self.gate_mlp(x).view(B, T, H, 3).permute(0, 2, 1, 3)
        # the projection's [B,T,H,dk] storage as it is (the kernels take any row strides)
        qk = q if _ops._rows_ok(q) else q.contiguous()
        o = NSACore.apply(qk, k_cmp, v_cmp, block_ends, k_sel.transpose(-1, -2), v_sel, indices,
                          k_win.transpose(-1, -2), v_win, gate_logits, self.scale, c)
        o = o.transpose(1, 2).reshape(B, T, H * dv)
        out = self.dropout(self.o_proj(o))
        info = None
        if output_attentions:
            with torch.no_grad():  # the activated gates, as returned by the reference
                gates = (torch.softmax(gate_logits, dim=-1) if c.gate_mode == "softmax"
                         else torch.sigmoid(gate_logits))
            info = {"compression_scores": p_cmp, "selection_scores": p_slc, "selected_indices": indices,
                    "gates": gates.permute(0, 2, 1, 3)}
        return out, info
