"""Write golden input/output vectors from the reference implementation.

Run in the build container only (the reference is not available on GPU boxes):
    python tests/golden/make_golden.py /root/reference

It imports the reference's pure-torch code (nsa/kernels.py's NSAAttention in eval mode,
whose branches run nsa/reference.py on the CPU in float64, and its selection
functions) for the parts no closed form pins exactly: the Eq. 8 -> 9 -> 10 -> top-n
pipeline with its fp32 rounding and tie order, compress_tokens, and the eval-mode
module output.  Only data is written (fixtures/*.npz); nothing from the reference is
kept under tests/.
"""
import sys
from pathlib import Path

import numpy as np
import torch

REF = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
sys.path.insert(0, str(REF))
from nsa.kernels import (NSAAttention, NSAConfig, derive_selection_from_compression_per_timestep,  # noqa: E402
                         select_top_k_blocks_per_query_with_gqa)

OUT = Path(__file__).resolve().parent / "fixtures"
OUT.mkdir(exist_ok=True)


def module_case(name, seed, B, T, **cfg_kw):
    torch.manual_seed(seed)
    cfg = NSAConfig(**cfg_kw)
    m = NSAAttention(cfg).eval()
    x = torch.randn(B, T, cfg.d_model)
    with torch.no_grad():
        out, info = m(x, output_attentions=True)
        q = m.q_proj(x).view(B, T, cfg.n_heads, cfg.head_dim_qk).transpose(1, 2)
        kcomp = m.k_compress(x).view(B, T, cfg.n_kv_groups, cfg.head_dim_qk).transpose(1, 2)
        vcomp = m.v_compress(x).view(B, T, cfg.n_kv_groups, cfg.head_dim_v).transpose(1, 2)
        kc, vc, be, nact = m.compress_tokens(kcomp, vcomp)
    arrs = {f"param/{k}": v.detach().numpy() for k, v in m.state_dict().items()}
    arrs.update({
        "x": x.numpy(), "out": out.numpy(), "q": q.numpy(), "k_comp_in": kcomp.numpy(), "v_comp_in": vcomp.numpy(),
        "k_cmp": kc.numpy(), "v_cmp": vc.numpy(), "block_ends": be.numpy(), "n_actual": np.int64(nact),
        "compression_scores": info["compression_scores"].numpy(), "selection_scores": info["selection_scores"].numpy(),
        "selected_indices": info["selected_indices"].numpy(), "gates": info["gates"].numpy(),
    })
    cfg_arr = {f"cfg/{k}": np.asarray(getattr(cfg, k)) for k in
               ("d_model", "head_dim_qk", "head_dim_v", "l", "d", "l_prime", "n", "include_fixed_in_selection",
                "n_fixed", "w", "n_heads", "n_kv_groups")}
    cfg_arr["cfg/gate_mode"] = np.asarray(cfg.gate_mode)
    arrs.update(cfg_arr)
    np.savez_compressed(OUT / f"{name}.npz", **arrs)
    print("wrote", name, {k: v.shape for k, v in arrs.items() if not k.startswith(("param/", "cfg/"))})


def heads_case(name, seed, B, T, **cfg_kw):
    """Selection at the paper's head shapes (dk = 192, 16 query heads per group): only
    what the Eq. 8 -> top-n pipeline reads and writes is kept (q, K_cmp, block_ends,
    selection scores and indices), not the module's parameters."""
    torch.manual_seed(seed)
    cfg = NSAConfig(**cfg_kw)
    m = NSAAttention(cfg).eval()
    x = torch.randn(B, T, cfg.d_model)
    with torch.no_grad():
        _, info = m(x, output_attentions=True)
        q = m.q_proj(x).view(B, T, cfg.n_heads, cfg.head_dim_qk).transpose(1, 2)
        kcomp = m.k_compress(x).view(B, T, cfg.n_kv_groups, cfg.head_dim_qk).transpose(1, 2)
        vcomp = m.v_compress(x).view(B, T, cfg.n_kv_groups, cfg.head_dim_v).transpose(1, 2)
        kc, _, be, _ = m.compress_tokens(kcomp, vcomp)
    arrs = {"q": q.contiguous().numpy(), "k_cmp": kc.numpy(), "block_ends": be.numpy(),
            "selection_scores": info["selection_scores"].numpy(), "selected_indices": info["selected_indices"].numpy()}
    for k in ("d_model", "head_dim_qk", "head_dim_v", "l", "d", "l_prime", "n", "include_fixed_in_selection",
              "n_fixed", "w", "n_heads", "n_kv_groups"):
        arrs[f"cfg/{k}"] = np.asarray(getattr(cfg, k))
    np.savez_compressed(OUT / f"{name}.npz", **arrs)
    print("wrote", name, {k: v.shape for k, v in arrs.items() if not k.startswith("cfg/")})


def topn_case(name, seed, B, H, G, T, nblk, n, l_prime, include_fixed, n_fixed, kind):
    g = torch.Generator().manual_seed(seed)
    if kind == "ties":
        # few distinct values -> many exact ties among blocks
        scores = torch.randint(0, 4, (B, H, T, nblk), generator=g).float() / 4
    elif kind == "causal":
        # scores zero past each row's causal frontier (as Eq. 8 produces)
        scores = torch.rand(B, H, T, nblk, generator=g)
        frontier = (torch.arange(T) // l_prime).view(1, 1, T, 1)
        scores = torch.where(torch.arange(nblk).view(1, 1, 1, nblk) <= frontier, scores, torch.zeros(()))
    else:
        scores = torch.rand(B, H, T, nblk, generator=g)
    cfg = NSAConfig(n_heads=H, n_kv_groups=G, n=n, l_prime=l_prime, d=16, l=32,
                    include_fixed_in_selection=include_fixed, n_fixed=n_fixed)
    idx = select_top_k_blocks_per_query_with_gqa(scores, cfg)
    np.savez_compressed(OUT / f"{name}.npz", scores=scores.numpy(), indices=idx.numpy(),
                        meta=np.array([G, n, l_prime, int(include_fixed), n_fixed]))
    print("wrote", name, idx.shape)


def eq9_case(name, seed, B, H, T, NB):
    g = torch.Generator().manual_seed(seed)
    p = torch.rand(B, H, T, NB, generator=g)
    p = p / p.sum(-1, keepdim=True)
    cfg = NSAConfig(l=32, d=16, l_prime=64)
    sel = derive_selection_from_compression_per_timestep(p, cfg)
    np.savez_compressed(OUT / f"{name}.npz", p_cmp=p.numpy(), p_slc=sel.numpy())
    print("wrote", name, sel.shape)


if __name__ == "__main__":
    torch.set_num_threads(8)
    # config 1 of the benchmark plan (CPU plumbing), reduced d_model
    module_case("module_cfg1", 0, B=1, T=512, d_model=128, head_dim_qk=64, head_dim_v=64, n_heads=8, n_kv_groups=2,
                l=32, d=16, l_prime=64, n=4, w=256)
    # odd length, softmax gates, no fixed blocks, l' = 32
    module_case("module_odd_softmax", 1, B=2, T=133, d_model=64, head_dim_qk=32, head_dim_v=32, n_heads=4,
                n_kv_groups=2, l=16, d=8, l_prime=32, n=3, w=40, gate_mode="softmax", include_fixed_in_selection=False)
    # T shorter than one compression block: fallback paths
    module_case("module_short", 2, B=1, T=24, d_model=64, head_dim_qk=32, head_dim_v=32, n_heads=4, n_kv_groups=1,
                l=32, d=16, l_prime=64, n=4, w=16)
    # the paper's head shapes: dk = 192, dv = 128, 16 query heads per KV group
    heads_case("heads_paper", 7, B=1, T=512, d_model=64, head_dim_qk=192, head_dim_v=128, n_heads=16,
               n_kv_groups=1, l=32, d=16, l_prime=64, n=5, w=128)
    topn_case("topn_ties_fixed", 3, B=2, H=8, G=2, T=256, nblk=8, n=5, l_prime=32, include_fixed=True, n_fixed=3,
              kind="ties")
    topn_case("topn_ties_nofixed", 4, B=1, H=4, G=4, T=64, nblk=16, n=6, l_prime=16, include_fixed=False, n_fixed=0,
              kind="ties")
    topn_case("topn_causal_nexceeds", 5, B=1, H=4, G=1, T=512, nblk=8, n=16, l_prime=64, include_fixed=True,
              n_fixed=3, kind="causal")
    eq9_case("eq9_random", 6, B=1, H=2, T=16, NB=37)
