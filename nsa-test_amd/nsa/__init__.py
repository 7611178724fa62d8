"""Native Sparse Attention (NSA) for AMD Instinct MI355X (gfx950).

Drop-in replacement for the ``nsa`` package of Noumena-Network/NSA-Test
(nsa/__init__.py:13-37): the same exported names, backed by hand-written HIP kernels
in libnsa_hip.so instead of Triton.

Based on "Native Sparse Attention: Hardware-Aligned and Natively Trainable Sparse
Attention" (arXiv:2502.11089).
"""
from .kernels import (
    CompressionAttention,
    GatedMix,
    NSAAttention,
    NSACore,
    NSAKVCache,
    NSAConfig,
    SelectionAttention,
    SlidingWindowAttention,
    _nsa_compression_bwd_kernel,
    _nsa_compression_fwd_kernel,
    _nsa_sliding_window_bwd_kernel,
    _nsa_sliding_window_fwd_kernel,
    _nsa_sparse_selection_bwd_kernel,
    _nsa_sparse_selection_fwd_kernel,
    derive_selection_from_compression_per_timestep,
    score_and_select,
    select_top_k_blocks_per_query_with_gqa,
)

__version__ = "1.0.0"

__all__ = [
    "NSAConfig",
    "NSAAttention",
    "_nsa_sliding_window_fwd_kernel",
    "_nsa_sliding_window_bwd_kernel",
    "_nsa_compression_fwd_kernel",
    "_nsa_compression_bwd_kernel",
    "_nsa_sparse_selection_fwd_kernel",
    "_nsa_sparse_selection_bwd_kernel",
]
