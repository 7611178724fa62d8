"""ctypes binding of libnsa_hip.so (the C ABI declared in include/nsa_hip.h).

The library is loaded lazily on first use.  There is no other implementation of
these operators: if the shared library is missing or cannot be loaded, every call
raises instead of falling back to anything.
"""
from __future__ import annotations

import ctypes
import threading
from ctypes import c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libnsa_hip.so")
ABI_VERSION = 5

NSA_F32 = 0
NSA_BF16 = 1

NSA_OK = 0
NSA_ERR_INVALID = 1
NSA_ERR_UNSUPPORTED = 2
NSA_ERR_LAYOUT = 3
NSA_ERR_WORKSPACE = 4
NSA_ERR_HIP = 5

_P, _F, _I, _L, _Z = c_void_p, c_float, c_int, c_int64, c_size_t

# name -> (restype, argtypes) for every exported symbol
_S22 = [_L] * 22
_S26 = [_L] * 26
_S12 = [_L] * 12
SIGNATURES = {
    "nsa_abi_version": (_I, []),
    "nsa_last_error": (ctypes.c_char_p, []),
    "nsa_head_dims_supported": (_I, [_I, _I, _I]),
    "nsa_fwd_workspace_size": (_Z, [_I] * 11),
    "nsa_bwd_workspace_size": (_Z, [_I] * 12),
    "nsa_bwd_dq_deferrable": (_I, [_I] * 12),
    "nsa_sliding_window_fwd": (_I, [_P, _P, _P, _P, _F, _P, _P, *_S22, *[_I] * 7, _I, _P, _Z, _P]),
    "nsa_sliding_window_bwd": (
        _I, [_P, _P, _P, _P, _P, _F, _P, _P, *_S22, _P, _P, _P, *_S12, *[_I] * 7, _I, _P, _Z, _P]),
    "nsa_compression_fwd": (_I, [_P, _P, _P, _P, _P, _F, _P, _P, *_S22, *[_I] * 7, _I, _P, _Z, _P]),
    "nsa_compression_bwd": (
        _I, [_P, _P, _P, _P, _P, _P, _F, _P, _P, *_S22, _P, _P, _P, *_S12, *[_I] * 7, _I, _P, _Z, _P]),
    "nsa_sparse_selection_fwd": (_I, [_P, _P, _P, _P, _P, _F, _P, _P, *_S26, *[_I] * 12, _I, _P, _Z, _P]),
    "nsa_sparse_selection_bwd": (
        _I, [_P, _P, _P, _P, _P, _P, _F, _P, _P, *_S26, _P, _P, _P, *_S12, *[_I] * 12, _I, _P, _Z, _P]),
}
# the allocation-free sliding-window forward: no workspace arguments
SIGNATURES["nsa_sliding_window_fwd_noalloc"] = (_I, SIGNATURES["nsa_sliding_window_fwd"][1][:-3] + [_P])
# the backward extensions: bwd_flags (int), delta_in, row_gate, row_dot (pointers)
# before the workspace
for _n in ("nsa_sliding_window_bwd", "nsa_compression_bwd", "nsa_sparse_selection_bwd"):
    _r, _a = SIGNATURES[_n]
    SIGNATURES[_n + "_ex"] = (_r, [*_a[:-3], _I, _P, _P, _P, *_a[-3:]])
# the sliding-window backward paired with a deferred compression backward: its block
# ends, block count and workspace (pointer, bytes) before the workspace
_r, _a = SIGNATURES["nsa_sliding_window_bwd_ex"]
SIGNATURES["nsa_sliding_window_bwd_pair"] = (_r, [*_a[:-3], _P, _I, _P, _Z, *_a[-3:]])
# the forward / scoring decode extensions: q_offset (sliding also n_ctx_kv and the gated
# mix: mix_o0, mix_o1, mix_gates, mix_out, three strides) before the workspace
for _n, _extra in (("nsa_sliding_window_fwd", [_I, _I, _P, _P, _P, _P, _L, _L, _L]), ("nsa_compression_fwd", [_I]),
                   ("nsa_sparse_selection_fwd", [_I])):
    _r, _a = SIGNATURES[_n]
    SIGNATURES[_n + "_ex"] = (_r, [*_a[:-3], *_extra, *_a[-3:]])
SIGNATURES.update({
    "nsa_score_topn": (_I, [_P, _P, _P, _P, _P, _P, *[_L] * 12, *[_I] * 13, _F, _P, _Z, _P]),
    "nsa_score_topn_workspace_size": (_Z, [_I] * 7),
    "nsa_score_topn_ex": (_I, [_P, _P, _P, _P, _P, _P, *[_L] * 12, *[_I] * 13, _F, _I, _P, _Z, _P]),
    "nsa_timing_begin": (_I, [_I]),
    "nsa_timing_end": (_I, [_P, _P]),
    "nsa_gate_mix_fwd": (_I, [_P] * 3 + [_L] * 3 + [_P] + [_L] * 4 + [_P] + [_L] * 3 + [_I] * 6 + [_P]),
    "nsa_gate_mix_bwd": (_I, [_P] + [_L] * 3 + [_P] * 3 + [_L] * 3 + [_P] + [_L] * 4 + [_P] * 5 + [_I] * 6 + [_P]),
    "nsa_gate_act_fwd": (_I, [_P] + [_L] * 4 + [_P] + [_I] * 5 + [_P]),
    "nsa_gate_act_bwd": (_I, [_P] * 3 + [_L] * 4 + [_I] * 5 + [_P]),
    "nsa_mix_row_dots": (_I, [_P] * 4 + [_L] * 3 + [_P] + [_I] * 5 + [_P]),
    "nsa_compress_pool_fwd": (_I, [_P] * 5 + [_I] * 10 + [_P]),
    "nsa_compress_pool_bwd": (_I, [_P] * 7 + [_I] * 10 + [_P]),
    "nsa_wgrad_workspace_size": (_Z, [_I] * 3),
    "nsa_wgrad": (_I, [_P, _L, _P, _L, _I, _I, _I, _P, _L, _I, _P, _Z, _P]),
    "nsa_bwd_dkdv_plan": (_I, [_I] * 9 + [_P, _P]),
})

_lock = threading.Lock()
_lib = None


class NSAKernelError(RuntimeError):
    """A libnsa_hip.so entry point returned an error code."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed (code {code}): {msg}")
        self.code = code


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()' "
                f"or python nsa-test_amd/nsa/_build.py)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
        ver = lib.nsa_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"libnsa_hip.so ABI {ver}, expected {ABI_VERSION}: rebuild it")
        _lib = lib
        return lib


def exported_symbols() -> list[str]:
    """Symbols of SIGNATURES that the loaded library exports."""
    lib = load()
    return [n for n in SIGNATURES if hasattr(lib, n)]


def call(name: str, *args) -> None:
    lib = load()
    fn = getattr(lib, name)
    rc = fn(*args)
    if rc != NSA_OK:
        msg = lib.nsa_last_error().decode(errors="replace")
        raise NSAKernelError(name, rc, msg)


_SIZE_CACHE: dict = {}


def size(name: str, *args) -> int:
    """A workspace-size query (a pure function of its integer arguments: memoised)."""
    key = (name, *args)
    r = _SIZE_CACHE.get(key)
    if r is None:
        r = _SIZE_CACHE[key] = int(getattr(load(), name)(*args))
    return r


def dkdv_plan(branch: int, Z: int, H: int, G: int, Tq: int, Tkv: int, n_slots: int, lprime: int,
              window: int) -> dict:
    """The dK/dV schedule of a backward launch: work items per (batch, group) and the
    query-segment length."""
    items, seg = ctypes.c_int(0), ctypes.c_int(0)
    call("nsa_bwd_dkdv_plan", branch, Z, H, G, Tq, Tkv, n_slots, lprime, window,
         ctypes.cast(ctypes.pointer(items), c_void_p), ctypes.cast(ctypes.pointer(seg), c_void_p))
    return {"items_per_bg": items.value, "segment": seg.value}


# kernel ids of nsa_timing_begin
KID_FWD, KID_DQ, KID_DKDV, KID_REDUCE, KID_SCORE, KID_POOL_FWD, KID_POOL_BWD = 0, 3, 6, 9, 10, 11, 12


class KernelTimer:
    """Sum of the device time of every launch of one kernel inside a `with` block,
    from HIP events the library records on the launch stream."""

    def __init__(self, kernel_id: int):
        self.kernel_id = kernel_id
        self.ms = 0.0
        self.launches = 0

    def __enter__(self):
        call("nsa_timing_begin", self.kernel_id)
        return self

    def __exit__(self, *exc):
        ms = ctypes.c_double(0.0)
        n = ctypes.c_int(0)
        call("nsa_timing_end", ctypes.cast(ctypes.pointer(ms), c_void_p), ctypes.cast(ctypes.pointer(n), c_void_p))
        self.ms, self.launches = ms.value, n.value
        return False
