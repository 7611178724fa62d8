"""CPU tests of the host side: configuration semantics, the torch selection helpers,
the C ABI library (loads, exports every declared symbol) and the launch surface's
argument handling.  No GPU computation happens here."""
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import nsa
from nsa import _lib, _ops
from nsa.kernels import NSAConfig, derive_selection_from_compression_per_timestep, select_top_k_blocks_per_query_with_gqa
from conftest import ROOT, load_fixture


# ------------------------------------------------------------------- config
def test_config_defaults_and_normalisation():
    c = NSAConfig()
    assert (c.head_dim_qk, c.head_dim_v, c.l, c.d, c.l_prime, c.n, c.w) == (192, 128, 32, 16, 64, 16, 512)
    assert (c.n_fixed, c.n_dynamic, c.gate_mode) == (3, 13, "sigmoid")
    assert c.heads_per_group == 16 and c.head_dim_qk_padded == 256 and c.head_dim_v_padded == 128
    c2 = NSAConfig(include_fixed_in_selection=False)
    assert c2.n_fixed == 0 and c2.n_dynamic == 16
    assert NSAConfig(n=8, n_fixed=3).n_dynamic == 5
    for bad in (dict(n_heads=6, n_kv_groups=4), dict(l=30, d=16), dict(l_prime=40, d=16), dict(w=0),
                dict(gate_mode="tanh")):
        with pytest.raises(AssertionError):
            NSAConfig(**bad)


def test_exports_match_reference_surface():
    names = {"NSAConfig", "NSAAttention", "_nsa_sliding_window_fwd_kernel", "_nsa_sliding_window_bwd_kernel",
             "_nsa_compression_fwd_kernel", "_nsa_compression_bwd_kernel", "_nsa_sparse_selection_fwd_kernel",
             "_nsa_sparse_selection_bwd_kernel"}
    assert set(nsa.__all__) == names and nsa.__version__ == "1.0.0"
    for n in ("CompressionAttention", "SelectionAttention", "SlidingWindowAttention",
              "derive_selection_from_compression_per_timestep", "select_top_k_blocks_per_query_with_gqa"):
        assert hasattr(nsa.kernels, n)


def test_module_state_dict_keys_match_reference_layout():
    c = NSAConfig(d_model=64, head_dim_qk=32, head_dim_v=32, n_heads=4, n_kv_groups=2)
    m = nsa.NSAAttention(c)
    f = load_fixture("module_odd_softmax")
    ref_keys = {k[6:] for k in f.files if k.startswith("param/")}
    assert set(m.state_dict().keys()) == ref_keys


# ------------------------------------------------- torch selection helpers
@pytest.mark.parametrize("name", ["topn_ties_fixed", "topn_ties_nofixed", "topn_causal_nexceeds"])
def test_select_top_k_golden(name):
    g = load_fixture(name)
    G, n, lp, inc, nf = (int(x) for x in g["meta"])
    H = g["scores"].shape[1]
    cfg = NSAConfig(n_heads=H, n_kv_groups=G, n=n, l_prime=lp, d=16, l=32, include_fixed_in_selection=bool(inc),
                    n_fixed=nf)
    got = select_top_k_blocks_per_query_with_gqa(torch.tensor(g["scores"]), cfg)
    np.testing.assert_array_equal(got.numpy(), g["indices"])


@pytest.mark.parametrize("name", ["module_cfg1", "module_odd_softmax", "module_short"])
def test_eq9_eq10_golden(name):
    f = load_fixture(name)
    kw = {k[4:]: f[k].item() for k in f.files if k.startswith("cfg/")}
    cfg = NSAConfig(**kw)
    sel = derive_selection_from_compression_per_timestep(torch.tensor(f["compression_scores"]), cfg)
    np.testing.assert_array_equal(sel.numpy(), f["selection_scores"])
    idx = select_top_k_blocks_per_query_with_gqa(torch.tensor(f["selection_scores"]), cfg)
    np.testing.assert_array_equal(idx.numpy(), f["selected_indices"])


def test_select_top_k_known_answers():
    scores = torch.arange(5, dtype=torch.float32).view(1, 1, 1, 5).repeat(1, 2, 3, 1)
    cfg = NSAConfig(l_prime=2, d=1, n=3, n_heads=2, n_kv_groups=1, include_fixed_in_selection=False)
    assert select_top_k_blocks_per_query_with_gqa(scores, cfg)[0, 0, 0].tolist() == [4, 3, 2]
    cfg = NSAConfig(l_prime=2, d=1, n=3, n_heads=2, n_kv_groups=1, include_fixed_in_selection=True, n_fixed=3)
    idx = select_top_k_blocks_per_query_with_gqa(scores, cfg)
    assert idx[0, 0, 0].tolist() == [0, 4, 3] and idx[0, 0, 2].tolist() == [0, 1, 4]


# ----------------------------------------------------------- the C ABI library
def _declared_functions():
    text = (ROOT / "include" / "nsa_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = re.findall(r"^(?:int|size_t|const char\*)\s+(nsa_\w+)\s*\(([^;]*)\);", text, flags=re.M)
    return {name: [a.strip() for a in args.split(",") if a.strip() and a.strip() != "void"] for name, args in decls}


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    decls = _declared_functions()
    assert len(decls) >= 15
    for name in decls:
        assert hasattr(lib, name), f"{name} declared in include/nsa_hip.h but not exported"
    assert lib.nsa_abi_version() == _lib.ABI_VERSION
    assert lib.nsa_head_dims_supported(_lib.NSA_BF16, 192, 128) == 1
    assert lib.nsa_head_dims_supported(_lib.NSA_F32, 48, 48) == 0


def test_ctypes_signatures_match_header():
    decls = _declared_functions()
    for name, args in decls.items():
        assert name in _lib.SIGNATURES, name
        assert len(_lib.SIGNATURES[name][1]) == len(args), f"{name}: {len(_lib.SIGNATURES[name][1])} != {len(args)}"


def test_workspace_sizes():
    f = _lib.size("nsa_fwd_workspace_size", 0, _lib.NSA_BF16, 1, 64, 4, 8192, 8192, 192, 128, 0, 64)
    b = _lib.size("nsa_bwd_workspace_size", 0, _lib.NSA_F32, 1, 64, 4, 8192, 8192, 192, 128, 0, 64, 512)
    assert 0 < f < b
    # with >= 256 key tiles (Z*G*tiles) the sliding dK/dV adds straight into dK/dV:
    # a wider window needs no partials then (fp32: no stored dS)
    assert _lib.size("nsa_bwd_workspace_size", 0, _lib.NSA_F32, 1, 64, 4, 8192, 8192, 192, 128, 0, 64, 8192) == b
    # with fewer tiles a wider window spreads each key tile over more query segments
    b1 = _lib.size("nsa_bwd_workspace_size", 0, _lib.NSA_F32, 1, 16, 1, 8192, 8192, 192, 128, 0, 64, 512)
    assert _lib.size("nsa_bwd_workspace_size", 0, _lib.NSA_F32, 1, 16, 1, 8192, 8192, 192, 128, 0, 64, 8192) > b1
    # bf16 with whole 16-head groups: the sliding window's dS stored per (timestep, head
    # group, 32-key chunk it sees: min((w + 62) / 32, T / 32 + 1) of them, 1 KB each);
    # a window whose dS would exceed 6 GiB recomputes it instead (w = 8192: 8.6 GB)
    tp = 8192 + 64
    kv = 4 * tp * (2 * 192 + 128) * 2  # bf16 K rowfrag + K colfrag + V rowfrag copies
    b16 = _lib.size("nsa_bwd_workspace_size", 0, _lib.NSA_BF16, 1, 64, 4, 8192, 8192, 192, 128, 0, 64, 512)
    ds = 4 * 8192 * ((512 + 62) // 32) * 1024
    assert b16 - (b - kv) == ds
    assert _lib.size("nsa_bwd_workspace_size", 0, _lib.NSA_BF16, 1, 64, 4, 8192, 8192, 192, 128, 0, 64, 8192) == b16 - ds
    s = _lib.size("nsa_bwd_workspace_size", 2, _lib.NSA_BF16, 1, 64, 4, 8192, 8192, 192, 128, 16, 64, 1)
    assert s > f
    # selection, bf16, 16 heads per group: the stored dS (2 bytes per (row, slot, key of
    # the block)) and the CSR entries' slots (4 bytes per (group row, slot)); fp32 and
    # 3 heads per group keep the recomputing dQ kernel and neither buffer
    sf = _lib.size("nsa_bwd_workspace_size", 2, _lib.NSA_F32, 1, 64, 4, 8192, 8192, 192, 128, 16, 64, 1)
    tp = 8192 + 64  # re-packed K/V rows (a multiple of 64, plus 64 zero rows)
    kv16 = 4 * tp * (2 * 192 + 128) * 2  # K rowfrag + K colfrag + V rowfrag copies, bf16
    # fp32 partials are 4 bytes per (item, key, feature), bf16 ones 2: 1152 items per group
    # here (128 blocks + 8192 * 16 entries / 128-entry segments), 64 keys, dk + dv = 320
    part16 = 4 * 1152 * 64 * 320 * 2
    assert s - (sf - kv16 - part16) == 64 * 8192 * 16 * 64 * 2 + 4 * 8192 * 16 * 4
    s3 = _lib.size("nsa_bwd_workspace_size", 2, _lib.NSA_BF16, 1, 12, 4, 8192, 8192, 192, 128, 16, 64, 1)
    s3f = _lib.size("nsa_bwd_workspace_size", 2, _lib.NSA_F32, 1, 12, 4, 8192, 8192, 192, 128, 16, 64, 1)
    assert s3f - s3 > 0  # only the fp32 K/V copies are larger
    # the selection dS grows with the batch: past 6 GiB (here B=4 at the long shape,
    # 32 * 32768 * 16 * 64 * 2 B = 2.1 GB per batch entry) the backward recomputes it,
    # so neither the dS nor the CSR slot buffer is allocated
    def sel(Z, dt):
        return _lib.size("nsa_bwd_workspace_size", 2, dt, Z, 32, 2, 32768, 32768, 128, 128, 16, 64, 1)
    ds1 = 32 * 32768 * 16 * 64 * 2
    assert sel(1, _lib.NSA_BF16) >= ds1
    kvd = 2 * (32768 + 64) * 3 * 128 * 2  # bf16 vs fp32 K/V copies per batch entry
    partd = 2 * (512 + 32768 * 16 // 256) * 64 * 256 * 2  # bf16 vs fp32 partials per batch entry
    assert sel(3, _lib.NSA_BF16) - sel(3, _lib.NSA_F32) > 3 * ds1 - 3 * (kvd + partd)
    assert sel(4, _lib.NSA_F32) - sel(4, _lib.NSA_BF16) == 4 * (kvd + partd)
    # scoring: fp32 logits [Z*H][T][N rounded up to 64], then one int per 128-row tile of
    # a group's (timestep, head) rows, padded to 256 bytes
    sc = _lib.load().nsa_score_topn_workspace_size
    assert sc(1, 64, 4, 8192, 192, 511, 16) == 64 * 8192 * 512 * 4 + 4096
    assert sc(2, 8, 2, 100, 64, 5, 4) == 2 * 8 * 100 * 64 * 4 + 256
    assert sc(1, 8, 3, 100, 64, 5, 4) == 0  # H not a multiple of the groups


def test_error_codes_without_gpu_work():
    # validation happens before any launch: unsupported head dims, bad window
    lib = _lib.load()
    rc = lib.nsa_sliding_window_fwd(*([None] * 4), 1.0, None, None, *([0] * 22), 1, 1, 1, 8, 4, 48, 48,
                                    _lib.NSA_F32, None, 0, None)
    assert rc == _lib.NSA_ERR_UNSUPPORTED and b"head dims" in lib.nsa_last_error()
    # the backward extensions reject unknown bwd_flags bits before any other work
    import ctypes
    argt = _lib.SIGNATURES["nsa_sliding_window_bwd_ex"][1]
    args = [1.0 if t is ctypes.c_float else (None if t in (ctypes.c_void_p,) or hasattr(t, "contents") else 0)
            for t in argt]
    args[len(argt) - 7] = _ops.BWD_DQ_ACCUMULATE | _ops.BWD_DKDV_OVERWRITE | 8
    rc = lib.nsa_sliding_window_bwd_ex(*args)
    assert rc == _lib.NSA_ERR_INVALID and b"bwd_flags" in lib.nsa_last_error()
    # the paired sliding-window backward runs its own dQ and needs the compression
    # backward's workspace
    argt = _lib.SIGNATURES["nsa_sliding_window_bwd_pair"][1]
    args = [1.0 if t is ctypes.c_float else (None if t in (ctypes.c_void_p,) or hasattr(t, "contents") else 0)
            for t in argt]
    args[len(argt) - 11] = _ops.BWD_DQ_DEFER
    assert lib.nsa_sliding_window_bwd_pair(*args) == _lib.NSA_ERR_INVALID
    assert b"NSA_BWD_DQ_DEFER" in lib.nsa_last_error()
    args[len(argt) - 11] = 0
    assert lib.nsa_sliding_window_bwd_pair(*args) == _lib.NSA_ERR_INVALID
    assert b"cmp_workspace" in lib.nsa_last_error()
    assert _ops.kernel_dims(48, 48) == (64, 64) and _ops.kernel_dims(192, 128) == (192, 128)
    with pytest.raises(ValueError):
        _ops.kernel_dims(512, 64)


def test_dq_deferrable_query():
    # dQ can be deferred / paired exactly where the backward stores dS: bf16 at whole
    # 16-head groups (selection also needs l' a multiple of 64 and slots)
    def q(br, dt, H=64, G=4, slots=16, lp=64):
        return _lib.size("nsa_bwd_dq_deferrable", br, dt, 1, H, G, 8192, 8192 if br != 1 else 512, 192, 128, slots,
                         lp, 512)
    for br in (0, 1, 2):
        assert q(br, _lib.NSA_BF16) == 1
        assert q(br, _lib.NSA_F32) == 0
        assert q(br, _lib.NSA_BF16, H=32, G=4) == 0  # 8 heads per group
    assert q(2, _lib.NSA_BF16, lp=32) == 0 and q(2, _lib.NSA_BF16, slots=0) == 0
    assert q(2, _lib.NSA_BF16, G=0) == 0


def test_dkdv_segment_choice():
    # benchmark configuration 2 (sliding window 512, B=2, G=2, T=4096): 32 key tiles per
    # group see 639 query rows each; 160-row segments give 4 per tile, 512 items (two
    # full rounds over 256 CUs) where 128-row ones give 640 (a third, half-empty round)
    assert _lib.dkdv_plan(0, 2, 8, 2, 4096, 4096, 0, 64, 512) == {"items_per_bg": 128, "segment": 160}
    # the paper selection (4608 items at 128 entries) and a launch with >= 4096 items at
    # 256 entries (the long selection) keep 128 and 256
    assert _lib.dkdv_plan(2, 1, 64, 4, 8192, 8192, 16, 64, 1)["segment"] == 128
    assert _lib.dkdv_plan(2, 1, 32, 2, 32768, 32768, 16, 64, 1)["segment"] == 256
    # the paper compression: 256 and 128 entries tie at 512 entry-steps; the shorter wins
    assert _lib.dkdv_plan(1, 1, 64, 4, 8192, 512, 0, 64, 1)["segment"] == 128


def test_cpu_tensors_fail_loudly():
    q = torch.randn(1, 2, 8, 32)
    k = torch.randn(1, 1, 32, 8)
    v = torch.randn(1, 1, 8, 32)
    cfg = NSAConfig(d_model=32, head_dim_qk=32, head_dim_v=32, n_heads=2, n_kv_groups=1)
    with pytest.raises(RuntimeError, match="GPU"):
        nsa.SlidingWindowAttention.apply(q, k, v, 0.1, 4, cfg)
    out = torch.empty(1, 2, 8, 32)
    L = torch.empty(1, 2, 8)
    with pytest.raises(RuntimeError, match="GPU"):
        nsa._nsa_sliding_window_fwd_kernel[(1, 2)](
            q, k, v, out, 0.1, L, L, *q.stride(), k.stride(0), k.stride(1), k.stride(3), k.stride(2), *v.stride(),
            *out.stride(), *L.stride(), *L.stride(), Z=1, H=2, N_KV_GROUPS=1, N_CTX=8, WINDOW_SIZE=4,
            HEAD_DIM_QK=32, HEAD_DIM_V=32, BLOCK_M=32, BLOCK_N=32)


def test_launcher_rejects_out_of_storage_strides():
    """Strides that would address memory outside the tensor are refused before any
    launch (torch's view bounds check), where the reference would read past it."""
    q = torch.randn(1, 2, 64, 32)
    k = torch.randn(1, 2, 32, 64)
    v = torch.randn(1, 2, 64, 32)
    out = torch.empty(1, 2, 64, 32)
    L = torch.empty(1, 2, 64)
    with pytest.raises(RuntimeError, match="out of bounds"):
        nsa._nsa_sliding_window_fwd_kernel[(1, 2)](
            q, k, v, out, 0.1, L, L, *q.stride(), *k.stride(), *v.stride(), *out.stride(), *L.stride(), *L.stride(),
            Z=1, H=2, N_KV_GROUPS=2, N_CTX=64, WINDOW_SIZE=16, HEAD_DIM_QK=32, HEAD_DIM_V=32, BLOCK_M=32,
            BLOCK_N=32)


def test_split_cols_gradient():
    """compress_tokens splits the first MLP weight into its key and position columns
    with one autograd function whose backward concatenates the two gradients: checked
    against finite differences, and with one part unused (its columns get zeros)."""
    from nsa.kernels import _SplitCols
    W = torch.randn(5, 9, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda w: _SplitCols.apply(w, 3), (W,))
    a, b = _SplitCols.apply(W, 3)
    (a * a).sum().backward()
    assert torch.equal(W.grad[:, 3:], torch.zeros(5, 6, dtype=torch.float64))
    assert torch.allclose(W.grad[:, :3], 2 * W.detach()[:, :3])


def test_cached_block_ends_survive_inference_mode():
    """The block_ends cache is filled outside inference mode: a tensor first built by an
    eval step under torch.inference_mode() can be saved for a later training backward."""
    from nsa.kernels import _block_ends
    with torch.inference_mode():
        be = _block_ends(64, 37, 16, 32, torch.device("cpu"))
    assert not be.is_inference()
    assert be[:37].tolist() == [i * 16 + 31 for i in range(37)] and set(be[37:].tolist()) == {999999}


def test_compression_stored_ds_block_limit():
    """bf16 compression with whole 16-head groups stores dS while its dQ pass can stage
    every 32-key chunk's first block end in LDS (at most 2048 chunks = 65536 blocks); past
    that the backward recomputes dS in its dQ kernel and allocates no dS buffer."""
    def args(nb, dt):
        return (1, dt, 1, 16, 1, 64, nb, 64, 64, 0, 64, 1)
    assert _lib.size("nsa_bwd_dq_deferrable", *args(65536, _lib.NSA_BF16)) == 1
    assert _lib.size("nsa_bwd_dq_deferrable", *args(65537, _lib.NSA_BF16)) == 0
    # the dS buffer: one 1 KB fragment per (timestep, head group, 32-key chunk)
    ds = 64 * (65536 // 32) * 1024
    stored = _lib.size("nsa_bwd_workspace_size", *args(65536, _lib.NSA_BF16))
    recomputed = _lib.size("nsa_bwd_workspace_size", *args(65537, _lib.NSA_BF16))
    assert stored - recomputed >= ds - 2 * 1024 * 1024  # one more block changes the rest little
