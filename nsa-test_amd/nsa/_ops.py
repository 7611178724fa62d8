"""Tensor-level wrappers over the C ABI of libnsa_hip.so.

All tensors are *logical views* with the reference's meaning:
    q      [Z, H, Tq, dk]          out / dO / dq  [Z, H, Tq, dv|dk]
    k      [Z, G, Tkv, dk]  (the (z, g, time, dk) view of a [B, G, dk, T] tensor)
    v      [Z, G, Tkv, dv]          dk / dv        [Z, G, Tkv, dk|dv]
    L, M   [Z, H, Tq] fp32
Views may have any strides; the library honours them where it can, and this module
supplies compact copies where the kernels need unit-stride rows (Q, Out, dO, dQ).
Head widths without a compiled kernel are zero-padded to the next compiled pair.
"""
from __future__ import annotations

import ctypes

import torch
import torch.nn.functional as F

from . import _lib

SLIDING, COMPRESSION, SELECTION = 0, 1, 2
# bwd_flags bits of the backward extension entry points (include/nsa_hip.h)
BWD_DQ_ACCUMULATE, BWD_DKDV_OVERWRITE, BWD_DQ_DEFER = 1, 2, 4
HEAD_DIM_PAIRS = ((32, 32), (64, 64), (128, 128), (192, 128))


def _dtype_code(dt: torch.dtype) -> int:
    return _lib.NSA_F32 if dt == torch.float32 else _lib.NSA_BF16


def compute_dtype(dt: torch.dtype) -> torch.dtype:
    """Element type the kernels run in for inputs of dtype `dt`."""
    return dt if dt in (torch.float32, torch.bfloat16) else torch.float32


def kernel_dims(dk: int, dv: int) -> tuple[int, int]:
    for a, b in HEAD_DIM_PAIRS:
        if a >= dk and b >= dv:
            return a, b
    raise ValueError(f"head dims dk={dk} dv={dv} exceed the largest compiled pair {HEAD_DIM_PAIRS[-1]}")


def _as(t: torch.Tensor, dt: torch.dtype) -> torch.Tensor:
    # t in dtype dt (a dtype test is cheaper than a no-op Tensor.to on the host path)
    return t if t.dtype == dt else t.to(dt)


def _rows_ok(t: torch.Tensor) -> bool:
    es = t.element_size()
    if t.stride(-1) != 1 and t.shape[-1] > 1:
        return False
    if t.data_ptr() % 16:
        return False
    return all((s * es) % 16 == 0 for s in t.stride()[:-1])


def _rows(t: torch.Tensor) -> torch.Tensor:
    return t if _rows_ok(t) else t.contiguous()


def _pad_last(t: torch.Tensor, width: int) -> torch.Tensor:
    return t if t.shape[-1] == width else F.pad(t, (0, width - t.shape[-1]))


def _stream(dev: torch.device) -> ctypes.c_void_p:
    # the raw handle of the device's current stream (the Stream object is not needed)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    return ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(idx))


def _check_device(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("NSA kernels run on the GPU only: got a tensor on " + str(t.device))


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _branch_extra(branch, Tkv, block_ends, indices, lprime):
    """(n_ctx_kv_or_blocks, n_slots, lprime) for the workspace query."""
    if branch == SELECTION:
        return indices.shape[-1], lprime
    return 0, 64


def attn_fwd(branch: int, q, k, v, scale: float, *, window: int = 0, block_ends=None, indices=None,
             lprime: int = 64, causal: bool = True, fallback: bool = False, out=None, L=None, M=None,
             q_offset: int = 0, mix=None):
    """Forward of one NSA branch.  Returns (out, L, M); `out`, `L`, `M` are written in
    place when given (with their own strides).  q_offset: absolute position of query row
    0 in the key sequence (decode past a cache; the sliding window then takes its key
    length from k).  mix (sliding only): (o0, o1, gates, mix_out) -- the kernel also
    writes mix_out = gates[0] o0 + gates[1] o1 + gates[2] out, with o0 / o1 the other two
    branch outputs (compute dtype, out's shape and strides: pass `out` too), gates fp32
    contiguous [3, Z, H, Tq] and mix_out any [Z, H, Tq, dv] view with unit-stride rows."""
    _check_device(q, k, v, block_ends, indices, out, L, M)
    Z, H, Tq, dk = q.shape
    G, Tkv = k.shape[1], k.shape[2]
    dv = v.shape[-1]
    dev = q.device
    cdt = compute_dtype(q.dtype)
    DK, DV = kernel_dims(dk, dv)
    qk = _rows(_pad_last(_as(q, cdt), DK))
    kk = _pad_last(_as(k, cdt), DK)
    vk = _pad_last(_as(v, cdt), DV)
    direct_out = out is not None and out.dtype == cdt and dv == DV and _rows_ok(out)
    o = out if direct_out else torch.empty(Z, H, Tq, DV, device=dev, dtype=cdt)
    Lk = L if L is not None else torch.empty(Z, H, Tq, device=dev, dtype=torch.float32)
    Mk = M if M is not None else torch.empty(Z, H, Tq, device=dev, dtype=torch.float32)
    n_slots = indices.shape[-1] if branch == SELECTION else 0
    ws_bytes = _lib.size("nsa_fwd_workspace_size", branch, _dtype_code(cdt), Z, H, G, Tq, Tkv, DK, DV, n_slots,
                         lprime)
    ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    dt = _dtype_code(cdt)
    common_strides = [*qk.stride(), *kk.stride(), *vk.stride(), *o.stride()]
    lm_strides = [*Lk.stride(), *Mk.stride()]
    st = _stream(dev)
    if q_offset < 0:
        raise ValueError("q_offset must be >= 0")
    # the reference-interface entry points, or their decode extensions
    dec = q_offset != 0 or (branch == SLIDING and (Tq != Tkv or mix is not None))
    sfx, tail = ("_ex", (int(q_offset), _ptr(ws), ws.numel(), st)) if dec else ("", (_ptr(ws), ws.numel(), st))
    if mix is not None and (branch != SLIDING or not direct_out or any(
            t.dtype != cdt or t.stride() != o.stride() for t in mix[:2])):
        raise ValueError("mix needs the sliding branch, `out` in the compute dtype and o0 / o1 with out's strides")
    if branch == SLIDING:
        if dec:
            if mix is not None:
                o0, o1, gates, xo = mix
                if gates.dtype != torch.float32 or not gates.is_contiguous() or tuple(gates.shape) != (3, Z, H, Tq):
                    raise ValueError(f"mix gates must be contiguous fp32 [3, {Z}, {H}, {Tq}]")
                mixargs = (_ptr(o0), _ptr(o1), _ptr(gates), _ptr(xo), *xo.stride()[:3])
            else:
                mixargs = (_ptr(None), _ptr(None), _ptr(None), _ptr(None), 0, 0, 0)
            tail = (Tkv, int(q_offset), *mixargs, *tail[1:])
        _lib.call("nsa_sliding_window_fwd" + sfx, _ptr(qk), _ptr(kk), _ptr(vk), _ptr(o), float(scale), _ptr(Lk),
                  _ptr(Mk), *common_strides, *lm_strides, Z, H, G, Tq, int(window), DK, DV, dt, *tail)
    elif branch == COMPRESSION:
        be = block_ends.to(torch.int32).contiguous()
        _lib.call("nsa_compression_fwd" + sfx, _ptr(qk), _ptr(kk), _ptr(vk), _ptr(be), _ptr(o), float(scale),
                  _ptr(Lk), _ptr(Mk), *common_strides, *lm_strides, Z, H, G, Tq, Tkv, DK, DV, dt, *tail)
    else:
        idx = indices if indices.dtype in (torch.int32, torch.int64) else indices.to(torch.int64)
        _lib.call("nsa_sparse_selection_fwd" + sfx, _ptr(qk), _ptr(kk), _ptr(vk), _ptr(idx), _ptr(o), float(scale),
                  _ptr(Lk), _ptr(Mk), *common_strides, *idx.stride(), *lm_strides, Z, H, G, Tq, Tkv, n_slots,
                  int(lprime), int(bool(causal)), int(idx.dtype == torch.int64), int(bool(fallback)), DK, DV, dt,
                  *tail)
    if direct_out:
        return o, Lk, Mk
    res = o[..., :dv]
    if out is not None:
        out.copy_(res)
        return out, Lk, Mk
    return (res if q.dtype == cdt else res.to(q.dtype)), Lk, Mk


class DeferredDq:
    """What a compression backward run with its dQ deferred leaves for the sliding-window
    backward that adds that dQ in its own dQ pass: the workspace holding the stored dS
    and re-packed K^T, and the block ends (held here until the paired call)."""

    __slots__ = ("ws", "block_ends", "n_blocks")

    def __init__(self):
        self.ws = self.block_ends = None
        self.n_blocks = 0


def dq_deferrable(branch: int, q, k, v, n_slots: int = 0, lprime: int = 64, window: int = 0) -> bool:
    """Whether this branch's backward stores dS (bf16, whole 16-head groups), so that its
    dQ can be deferred / paired; q [Z,H,Tq,dk], k [Z,G,Tkv,dk], v [Z,G,Tkv,dv] views."""
    Z, H, Tq, dkw = q.shape
    DK, DV = kernel_dims(dkw, v.shape[-1])
    return _lib.size("nsa_bwd_dq_deferrable", branch, _dtype_code(compute_dtype(q.dtype)), Z, H, k.shape[1], Tq,
                     k.shape[2], DK, DV, n_slots, lprime, int(window) if branch == SLIDING else 1) == 1


def attn_bwd(branch: int, q, k, v, o, do, L, M, scale: float, *, window: int = 0, block_ends=None, indices=None,
             lprime: int = 64, causal: bool = True, fallback: bool = False, dq=None, dk=None, dv=None,
             dq_accumulate: bool = False, delta=None, row_gate=None, row_dot=None, dkdv_overwrite: bool = False,
             defer_dq: DeferredDq | None = None, pair: DeferredDq | None = None):
    """Backward of one NSA branch.  dq is overwritten (added to when dq_accumulate, which
    needs dq), dk / dv ([Z,G,Tkv,*] logical views) are accumulated into, or overwritten
    when dkdv_overwrite (allocated when not given: the kernels then write every element,
    so no zero fill is needed).  delta: optional precomputed row sums sum_d o * do [Z,H,Tq]
    (fp32), used instead of reading o.  row_gate: optional fp32 contiguous [Z,H,Tq]; the
    branch's output gradient is then row_gate * do.  row_dot: optional fp32 contiguous
    [Z,H,Tq] that receives sum_d do * o per row.  Sliding window: k / v may hold more
    keys than q has rows (none past the last row is visible: their gradient is zero), not
    fewer.  defer_dq (compression, where dq_deferrable): dq is left as it is and the state
    its dQ needs is stored into the given DeferredDq, for `pair`.  pair (sliding window,
    same q / do / scale): that compression backward's dQ is added in this call's dQ pass,
    so both reach dq with one read and write of it (dq must be written in place).
    Returns (dq, dk, dv)."""
    if dq_accumulate and dq is None:
        raise ValueError("dq_accumulate needs the dq tensor to add to")
    if defer_dq is not None and branch != COMPRESSION:
        raise ValueError("defer_dq is for the compression branch")
    if pair is not None and (branch != SLIDING or pair.ws is None):
        raise ValueError("pair needs the sliding-window branch and a deferred compression backward")
    _check_device(q, k, v, o, do, L, M, block_ends, indices, dq, dk, dv)
    Z, H, Tq, dkw = q.shape
    G, Tkv = k.shape[1], k.shape[2]
    dvw = v.shape[-1]
    if branch == SLIDING and Tkv < Tq:
        raise ValueError(f"sliding window backward: {Tkv} keys for {Tq} query rows (needs at least as many)")
    dev = q.device
    cdt = compute_dtype(q.dtype)
    DK, DV = kernel_dims(dkw, dvw)
    qk = _rows(_pad_last(_as(q, cdt), DK))
    kk = _pad_last(_as(k, cdt), DK)
    vk = _pad_last(_as(v, cdt), DV)
    # O and dO are read with one set of strides (as the reference kernels do): kept as
    # they are when they already share unit-stride, aligned rows
    ok = _pad_last(_as(o, cdt), DV)
    dok = _pad_last(_as(do, cdt), DV)
    if ok.stride() != dok.stride() or not (_rows_ok(ok) and _rows_ok(dok)):
        ok, dok = ok.contiguous(), dok.contiguous()
    Lf = _as(L, torch.float32)
    Mf = _as(M, torch.float32)
    direct_dq = dq is not None and dq.dtype == cdt and dkw == DK and _rows_ok(dq)
    acc = bool(dq_accumulate) and direct_dq  # otherwise the sum is taken below
    dqk = dq if direct_dq else torch.empty(Z, H, Tq, DK, device=dev, dtype=cdt)
    direct_dk = dk is not None and dk.dtype == cdt and dkw == DK
    direct_dv = dv is not None and dv.dtype == cdt and dvw == DV
    # overwrite mode when the caller asks for it or both buffers are this call's own
    ow = bool(dkdv_overwrite) or (not direct_dk and not direct_dv)
    alloc = torch.empty if ow else torch.zeros
    dkk = dk if direct_dk else alloc(Z, G, Tkv, DK, device=dev, dtype=cdt)
    dvk = dv if direct_dv else alloc(Z, G, Tkv, DV, device=dev, dtype=cdt)
    n_slots = indices.shape[-1] if branch == SELECTION else 0
    ws_bytes = _lib.size("nsa_bwd_workspace_size", branch, _dtype_code(cdt), Z, H, G, Tq, Tkv, DK, DV, n_slots,
                         lprime, int(window) if branch == SLIDING else 1)
    ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    dt = _dtype_code(cdt)
    st = _stream(dev)
    s_main = [*qk.stride(), *kk.stride(), *vk.stride(), *ok.stride()]
    s_lm = [*Lf.stride(), *Mf.stride()]
    s_grad = [*dqk.stride(), *dkk.stride(), *dvk.stride()]
    # the reference-interface entry points, or their extensions when dQ is added to
    dl = None if delta is None else delta.to(torch.float32).contiguous()
    if dl is not None and tuple(dl.shape) != (Z, H, Tq):
        raise ValueError(f"delta must be [{Z}, {H}, {Tq}], got {tuple(dl.shape)}")
    for t in (row_gate, row_dot):
        if t is not None and (t.dtype != torch.float32 or not t.is_contiguous() or tuple(t.shape) != (Z, H, Tq)):
            raise ValueError(f"row_gate / row_dot must be contiguous fp32 [{Z}, {H}, {Tq}]")
    if (defer_dq is not None or pair is not None) and not direct_dq:
        raise ValueError("a deferred or paired dQ is written in place: dq must be given in the compute dtype "
                         "with unit-stride, 16-byte aligned rows")
    if acc or ow or dl is not None or row_gate is not None or row_dot is not None or defer_dq is not None:
        flags = (BWD_DQ_ACCUMULATE if acc else 0) | (BWD_DKDV_OVERWRITE if ow else 0)
        flags |= BWD_DQ_DEFER if defer_dq is not None else 0
        sfx, tail = "_ex", (flags, _ptr(dl), _ptr(row_gate), _ptr(row_dot), _ptr(ws), ws.numel(), st)
    else:
        sfx, tail = "", (_ptr(ws), ws.numel(), st)
    if pair is not None:
        flags = (BWD_DQ_ACCUMULATE if acc else 0) | (BWD_DKDV_OVERWRITE if ow else 0)
        sfx, tail = "_pair", (flags, _ptr(dl), _ptr(row_gate), _ptr(row_dot), _ptr(pair.block_ends), pair.n_blocks,
                              _ptr(pair.ws), pair.ws.numel(), _ptr(ws), ws.numel(), st)
    if branch == SLIDING:
        _lib.call("nsa_sliding_window_bwd" + sfx, _ptr(qk), _ptr(kk), _ptr(vk), _ptr(ok), _ptr(dok), float(scale),
                  _ptr(Lf), _ptr(Mf), *s_main, *s_lm, _ptr(dqk), _ptr(dkk), _ptr(dvk), *s_grad, Z, H, G, Tq,
                  int(window), DK, DV, dt, *tail)
    elif branch == COMPRESSION:
        be = block_ends.to(torch.int32).contiguous()
        _lib.call("nsa_compression_bwd" + sfx, _ptr(qk), _ptr(kk), _ptr(vk), _ptr(be), _ptr(ok), _ptr(dok), float(scale),
                  _ptr(Lf), _ptr(Mf), *s_main, *s_lm, _ptr(dqk), _ptr(dkk), _ptr(dvk), *s_grad, Z, H, G, Tq, Tkv,
                  DK, DV, dt, *tail)
        if defer_dq is not None:
            defer_dq.ws, defer_dq.block_ends, defer_dq.n_blocks = ws, be, Tkv
    else:
        idx = indices if indices.dtype in (torch.int32, torch.int64) else indices.to(torch.int64)
        _lib.call("nsa_sparse_selection_bwd" + sfx, _ptr(qk), _ptr(kk), _ptr(vk), _ptr(idx), _ptr(ok), _ptr(dok),
                  float(scale), _ptr(Lf), _ptr(Mf), *s_main, *idx.stride(), *s_lm, _ptr(dqk), _ptr(dkk), _ptr(dvk),
                  *s_grad, Z, H, G, Tq, Tkv, n_slots, int(lprime), int(bool(causal)), int(idx.dtype == torch.int64),
                  int(bool(fallback)), DK, DV, dt, *tail)
    if branch == SLIDING and Tkv > Tq and ow:
        # the sliding-window entry points know one length (N_CTX = Tq): keys past it are
        # visible to no query row, so their gradient is zero
        dkk[:, :, Tq:].zero_()
        dvk[:, :, Tq:].zero_()
    if not direct_dq:
        r = dqk[..., :dkw]
        if dq is not None and dq_accumulate:
            dq.add_(r.to(dq.dtype))
        elif dq is not None:
            dq.copy_(r)
        else:
            dq = r if q.dtype == cdt else r.to(q.dtype)
    if not direct_dk:
        r = dkk[..., :dkw]
        if dk is not None:
            dk.copy_(r) if dkdv_overwrite else dk.add_(r.to(dk.dtype))
        else:
            dk = r if q.dtype == cdt else r.to(q.dtype)
    if not direct_dv:
        r = dvk[..., :dvw]
        if dv is not None:
            dv.copy_(r) if dkdv_overwrite else dv.add_(r.to(dv.dtype))
        else:
            dv = r if q.dtype == cdt else r.to(q.dtype)
    return dq, dk, dv
