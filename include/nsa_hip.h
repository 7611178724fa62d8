/*
 * C ABI of libnsa_hip.so: the MI355X (gfx950) Native Sparse Attention hot path.
 *
 * Each attention entry point takes exactly the argument list of the Triton launch
 * it replaces in the reference (tensors, sm_scale, L, M, the stride groups, then the
 * constexpr shape parameters), followed by the element type, a caller-allocated
 * device workspace and the HIP stream.  Pointers are device pointers, strides are in
 * elements, exactly as torch reports them.  Nothing is allocated and no state is
 * kept; every call is asynchronous on `stream`.
 *
 * Conventions shared by every attention entry point
 *   - K is stored [B, G, dk, T] and the caller passes its strides as
 *     (z, g, time, dk), i.e. k.stride(0), k.stride(1), k.stride(3), k.stride(2).
 *     K, V, dK, dV accept any strides.
 *   - Q, Out, dOut and dQ need unit stride on the feature axis and 16-byte aligned
 *     rows (NSA_ERR_LAYOUT otherwise; the Python shim then passes a compact copy).
 *   - head_dim_qk / head_dim_v are the real widths.  Pairs without a compiled kernel
 *     return NSA_ERR_UNSUPPORTED (the shim zero-pads to a supported pair).
 *   - dK and dV are accumulated into (the caller zero-fills them, as in the
 *     reference); dQ is overwritten.
 *   - dtype: NSA_F32 or NSA_BF16 (Q/K/V/Out/dOut/dQ/dK/dV share it; L, M are fp32).
 *   - Work is deterministic: no floating-point atomics anywhere.
 * Return value: NSA_OK or an NSA_ERR_* code; nsa_last_error() describes the failure.
 */
#ifndef NSA_HIP_H
#define NSA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* nsa_stream_t; /* == hipStream_t */

enum { NSA_F32 = 0, NSA_BF16 = 1 };
enum {
  NSA_OK = 0,
  NSA_ERR_INVALID = 1,
  NSA_ERR_UNSUPPORTED = 2,
  NSA_ERR_LAYOUT = 3,
  NSA_ERR_WORKSPACE = 4,
  NSA_ERR_HIP = 5
};

/* bwd_flags bits of the backward extensions (nsa_*_bwd_ex) */
enum { NSA_BWD_DQ_ACCUMULATE = 1, NSA_BWD_DKDV_OVERWRITE = 2, NSA_BWD_DQ_DEFER = 4 };

/* ABI revision of this header. */
int nsa_abi_version(void);
/* Text of the last error raised on the calling thread ("" if none). */
const char* nsa_last_error(void);
/* 1 if a kernel exists for (dtype, dk, dv). */
int nsa_head_dims_supported(int dtype, int dk, int dv);

/* ---- workspace sizes (bytes) ------------------------------------------------
 * branch: 0 sliding, 1 compression, 2 selection.  n_ctx_kv is T for sliding and
 * selection and N_BLOCKS for compression; n_slots / block_size_selection are only
 * read for selection. */
size_t nsa_fwd_workspace_size(int branch, int dtype, int Z, int H, int n_kv_groups, int n_ctx_q, int n_ctx_kv,
                              int head_dim_qk, int head_dim_v, int n_slots, int block_size_selection);
size_t nsa_bwd_workspace_size(int branch, int dtype, int Z, int H, int n_kv_groups, int n_ctx_q, int n_ctx_kv,
                              int head_dim_qk, int head_dim_v, int n_slots, int block_size_selection,
                              int window_size);
/* No counterpart in the reference: 1 when the backward of this shape stores dS for its
 * dQ kernel (bf16, whole 16-head groups, dS within the size cap), so that its dQ can be
 * deferred (NSA_BWD_DQ_DEFER) and paired (nsa_sliding_window_bwd_pair); else 0.  Same
 * arguments as nsa_bwd_workspace_size. */
int nsa_bwd_dq_deferrable(int branch, int dtype, int Z, int H, int n_kv_groups, int n_ctx_q, int n_ctx_kv,
                          int head_dim_qk, int head_dim_v, int n_slots, int block_size_selection, int window_size);

/* ---- sliding window --------------------------------------------------------
 * Replaces _nsa_sliding_window_fwd_kernel (reference nsa/kernels.py:1151-1191) and
 * _nsa_sliding_window_bwd_kernel (nsa/kernels.py:1303-1363).  Key j is visible to
 * query t iff t - window_size < j <= t. */
int nsa_sliding_window_fwd(const void* Q, const void* K, const void* V, void* Out, float sm_scale, float* L, float* M,
                           int64_t stride_qz, int64_t stride_qh, int64_t stride_qm, int64_t stride_qk,
                           int64_t stride_kz, int64_t stride_kg, int64_t stride_kn, int64_t stride_kk,
                           int64_t stride_vz, int64_t stride_vg, int64_t stride_vn, int64_t stride_vk,
                           int64_t stride_oz, int64_t stride_oh, int64_t stride_om, int64_t stride_ok,
                           int64_t stride_lz, int64_t stride_lh, int64_t stride_lm, int64_t stride_mz,
                           int64_t stride_mh, int64_t stride_mm, int Z, int H, int n_kv_groups, int n_ctx,
                           int window_size, int head_dim_qk, int head_dim_v, int dtype, void* workspace,
                           size_t workspace_bytes, nsa_stream_t stream);

int nsa_sliding_window_bwd(const void* Q, const void* K, const void* V, const void* Out, const void* dOut,
                           float sm_scale, const float* L, const float* M, int64_t stride_qz, int64_t stride_qh,
                           int64_t stride_qm, int64_t stride_qk, int64_t stride_kz, int64_t stride_kg,
                           int64_t stride_kn, int64_t stride_kk, int64_t stride_vz, int64_t stride_vg,
                           int64_t stride_vn, int64_t stride_vk, int64_t stride_oz, int64_t stride_oh,
                           int64_t stride_om, int64_t stride_ok, int64_t stride_lz, int64_t stride_lh,
                           int64_t stride_lm, int64_t stride_mz, int64_t stride_mh, int64_t stride_mm, void* dQ,
                           void* dK, void* dV, int64_t stride_dqz, int64_t stride_dqh, int64_t stride_dqm,
                           int64_t stride_dqk, int64_t stride_dkz, int64_t stride_dkg, int64_t stride_dkn,
                           int64_t stride_dkk, int64_t stride_dvz, int64_t stride_dvg, int64_t stride_dvn,
                           int64_t stride_dvk, int Z, int H, int n_kv_groups, int n_ctx, int window_size,
                           int head_dim_qk, int head_dim_v, int dtype, void* workspace, size_t workspace_bytes,
                           nsa_stream_t stream);

/* ---- compression -----------------------------------------------------------
 * Replaces _nsa_compression_fwd_kernel (nsa/kernels.py:1533-1574) and
 * _nsa_compression_bwd_kernel (nsa/kernels.py:1690-1751).  Compressed key i is
 * visible to query t iff Block_ends[i] <= t; rows with no visible key produce 0,
 * L = M = -inf.  Block_ends: int32, contiguous, N_BLOCKS entries. */
int nsa_compression_fwd(const void* Q, const void* K_compressed, const void* V_compressed, const int32_t* Block_ends,
                        void* Out, float sm_scale, float* L, float* M, int64_t stride_qz, int64_t stride_qh,
                        int64_t stride_qm, int64_t stride_qk, int64_t stride_kz, int64_t stride_kg,
                        int64_t stride_kn, int64_t stride_kk, int64_t stride_vz, int64_t stride_vg,
                        int64_t stride_vn, int64_t stride_vk, int64_t stride_oz, int64_t stride_oh,
                        int64_t stride_om, int64_t stride_ok, int64_t stride_lz, int64_t stride_lh,
                        int64_t stride_lm, int64_t stride_mz, int64_t stride_mh, int64_t stride_mm, int Z, int H,
                        int n_kv_groups, int n_ctx_q, int n_blocks, int head_dim_qk, int head_dim_v, int dtype,
                        void* workspace, size_t workspace_bytes, nsa_stream_t stream);

int nsa_compression_bwd(const void* Q, const void* K_blocks, const void* V_blocks, const int32_t* Block_ends,
                        const void* Out, const void* dOut, float sm_scale, const float* L, const float* M,
                        int64_t stride_qz, int64_t stride_qh, int64_t stride_qm, int64_t stride_qk,
                        int64_t stride_kz, int64_t stride_kg, int64_t stride_kn, int64_t stride_kk,
                        int64_t stride_vz, int64_t stride_vg, int64_t stride_vn, int64_t stride_vk,
                        int64_t stride_oz, int64_t stride_oh, int64_t stride_om, int64_t stride_ok,
                        int64_t stride_lz, int64_t stride_lh, int64_t stride_lm, int64_t stride_mz,
                        int64_t stride_mh, int64_t stride_mm, void* dQ, void* dK, void* dV, int64_t stride_dqz,
                        int64_t stride_dqh, int64_t stride_dqm, int64_t stride_dqk, int64_t stride_dkz,
                        int64_t stride_dkg, int64_t stride_dkn, int64_t stride_dkk, int64_t stride_dvz,
                        int64_t stride_dvg, int64_t stride_dvn, int64_t stride_dvk, int Z, int H, int n_kv_groups,
                        int n_ctx_q, int n_blocks, int head_dim_qk, int head_dim_v, int dtype, void* workspace,
                        size_t workspace_bytes, nsa_stream_t stream);

/* ---- top-n block selection -------------------------------------------------
 * Replaces _nsa_sparse_selection_fwd_kernel (nsa/kernels.py:594-654) and
 * _nsa_sparse_selection_bwd_kernel (nsa/kernels.py:836-906).  Block_indices is
 * [B, G, Tq, n_slots] (int32, or int64 when index_is_int64), -1 = empty slot; it
 * may be NULL when n_slots or n_ctx_q is 0 (nothing is read).
 * Key j is visible to query t iff (j <= t when is_causal) and j lies in one of the
 * row's blocks [idx*l', idx*l'+l').  Repeated indices count once.  With
 * all_invalid_fallback set, a row whose slots are all -1 uses block t / l' (the
 * autograd wrapper's rule, nsa/kernels.py:199-205).  block_size_selection must be
 * a multiple of 16. */
int nsa_sparse_selection_fwd(const void* Q, const void* K, const void* V, const void* Block_indices, void* Out,
                             float sm_scale, float* L, float* M, int64_t stride_qz, int64_t stride_qh,
                             int64_t stride_qm, int64_t stride_qk, int64_t stride_kz, int64_t stride_kg,
                             int64_t stride_kn, int64_t stride_kk, int64_t stride_vz, int64_t stride_vg,
                             int64_t stride_vn, int64_t stride_vk, int64_t stride_oz, int64_t stride_oh,
                             int64_t stride_om, int64_t stride_ok, int64_t stride_bz, int64_t stride_bg,
                             int64_t stride_bm, int64_t stride_bn, int64_t stride_lz, int64_t stride_lh,
                             int64_t stride_lm, int64_t stride_mz, int64_t stride_mh, int64_t stride_mm, int Z, int H,
                             int n_kv_groups, int n_ctx_q, int n_ctx_kv, int n_slots, int block_size_selection,
                             int is_causal, int index_is_int64, int all_invalid_fallback, int head_dim_qk,
                             int head_dim_v, int dtype, void* workspace, size_t workspace_bytes,
                             nsa_stream_t stream);

int nsa_sparse_selection_bwd(const void* Q, const void* K, const void* V, const void* Block_indices, const void* Out,
                             const void* dOut, float sm_scale, const float* L, const float* M, int64_t stride_qz,
                             int64_t stride_qh, int64_t stride_qm, int64_t stride_qk, int64_t stride_kz,
                             int64_t stride_kg, int64_t stride_kn, int64_t stride_kk, int64_t stride_vz,
                             int64_t stride_vg, int64_t stride_vn, int64_t stride_vk, int64_t stride_oz,
                             int64_t stride_oh, int64_t stride_om, int64_t stride_ok, int64_t stride_bz,
                             int64_t stride_bg, int64_t stride_bm, int64_t stride_bn, int64_t stride_lz,
                             int64_t stride_lh, int64_t stride_lm, int64_t stride_mz, int64_t stride_mh,
                             int64_t stride_mm, void* dQ, void* dK, void* dV, int64_t stride_dqz, int64_t stride_dqh,
                             int64_t stride_dqm, int64_t stride_dqk, int64_t stride_dkz, int64_t stride_dkg,
                             int64_t stride_dkn, int64_t stride_dkk, int64_t stride_dvz, int64_t stride_dvg,
                             int64_t stride_dvn, int64_t stride_dvk, int Z, int H, int n_kv_groups, int n_ctx_q,
                             int n_ctx_kv, int n_slots, int block_size_selection, int is_causal, int index_is_int64,
                             int all_invalid_fallback, int head_dim_qk, int head_dim_v, int dtype, void* workspace,
                             size_t workspace_bytes, nsa_stream_t stream);

/* Decode extensions (no counterpart in the reference): the forward entry points and
 * the scoring with the query rows placed at absolute positions q_offset ..
 * q_offset + n_ctx_q - 1 of the key sequence (row r of Q / Out / L / M / indices is
 * position q_offset + r; masks, fixed blocks and the all-invalid fallback use positions).
 * For single-token decode over a cache: n_ctx_q = 1, q_offset = cache length - 1.
 * The sliding-window form also takes the key length n_ctx_kv (the reference kernel
 * assumes n_ctx_kv = n_ctx) and, for the NSA module's forward (nsa/kernels.py:2429-2463),
 * a gated-mix epilogue: with mix_out not null it also writes
 *   mix_out[z,h,t,:] = g0 mix_o0[z,h,t,:] + g1 mix_o1[z,h,t,:] + g2 Out[z,h,t,:]
 * (fp32 sum of the stored values, rounded once), g_k = mix_gates[k,z,h,t] (contiguous
 * fp32 [3,Z,H,n_ctx]); mix_o0 / mix_o1 (the other two branch outputs) share Out's
 * strides, mix_out has its own (stride_x*, unit feature stride).  With q_offset = 0,
 * n_ctx_kv = n_ctx and mix_out null each behaves exactly as the entry point it extends. */
int nsa_sliding_window_fwd_ex(const void* Q, const void* K, const void* V, void* Out, float sm_scale, float* L, float* M,
                           int64_t stride_qz, int64_t stride_qh, int64_t stride_qm, int64_t stride_qk,
                           int64_t stride_kz, int64_t stride_kg, int64_t stride_kn, int64_t stride_kk,
                           int64_t stride_vz, int64_t stride_vg, int64_t stride_vn, int64_t stride_vk,
                           int64_t stride_oz, int64_t stride_oh, int64_t stride_om, int64_t stride_ok,
                           int64_t stride_lz, int64_t stride_lh, int64_t stride_lm, int64_t stride_mz,
                           int64_t stride_mh, int64_t stride_mm, int Z, int H, int n_kv_groups, int n_ctx,
                           int window_size, int head_dim_qk, int head_dim_v, int dtype,
                           int n_ctx_kv, int q_offset, const void* mix_o0, const void* mix_o1,
                           const float* mix_gates, void* mix_out, int64_t stride_xz, int64_t stride_xh,
                           int64_t stride_xm, void* workspace, size_t workspace_bytes, nsa_stream_t stream);

int nsa_compression_fwd_ex(const void* Q, const void* K_compressed, const void* V_compressed, const int32_t* Block_ends,
                        void* Out, float sm_scale, float* L, float* M, int64_t stride_qz, int64_t stride_qh,
                        int64_t stride_qm, int64_t stride_qk, int64_t stride_kz, int64_t stride_kg,
                        int64_t stride_kn, int64_t stride_kk, int64_t stride_vz, int64_t stride_vg,
                        int64_t stride_vn, int64_t stride_vk, int64_t stride_oz, int64_t stride_oh,
                        int64_t stride_om, int64_t stride_ok, int64_t stride_lz, int64_t stride_lh,
                        int64_t stride_lm, int64_t stride_mz, int64_t stride_mh, int64_t stride_mm, int Z, int H,
                        int n_kv_groups, int n_ctx_q, int n_blocks, int head_dim_qk, int head_dim_v, int dtype,
                        int q_offset, void* workspace, size_t workspace_bytes, nsa_stream_t stream);

int nsa_sparse_selection_fwd_ex(const void* Q, const void* K, const void* V, const void* Block_indices, void* Out,
                             float sm_scale, float* L, float* M, int64_t stride_qz, int64_t stride_qh,
                             int64_t stride_qm, int64_t stride_qk, int64_t stride_kz, int64_t stride_kg,
                             int64_t stride_kn, int64_t stride_kk, int64_t stride_vz, int64_t stride_vg,
                             int64_t stride_vn, int64_t stride_vk, int64_t stride_oz, int64_t stride_oh,
                             int64_t stride_om, int64_t stride_ok, int64_t stride_bz, int64_t stride_bg,
                             int64_t stride_bm, int64_t stride_bn, int64_t stride_lz, int64_t stride_lh,
                             int64_t stride_lm, int64_t stride_mz, int64_t stride_mh, int64_t stride_mm, int Z, int H,
                             int n_kv_groups, int n_ctx_q, int n_ctx_kv, int n_slots, int block_size_selection,
                             int is_causal, int index_is_int64, int all_invalid_fallback, int head_dim_qk,
                             int head_dim_v, int dtype, int q_offset, void* workspace, size_t workspace_bytes,
                             nsa_stream_t stream);

int nsa_score_topn_ex(const void* q, const void* k_cmp, const int32_t* Block_ends, int64_t* out_idx, float* p_cmp,
                   float* p_slc, int64_t stride_qz, int64_t stride_qh, int64_t stride_qm, int64_t stride_qk,
                   int64_t stride_kz, int64_t stride_kg, int64_t stride_kk, int64_t stride_kn, int64_t stride_iz,
                   int64_t stride_ig, int64_t stride_im, int64_t stride_in, int Z, int H, int n_kv_groups, int n_ctx,
                   int head_dim_qk, int n_blocks, int l, int d, int l_prime, int n, int include_fixed, int n_fixed,
                   int dtype, float scale,
                   int q_offset, void* workspace, size_t workspace_bytes, nsa_stream_t stream);

/* Extensions (no counterpart in the reference): the three backward entry points above
 * with two more arguments, for callers that run the three branches over one query
 * tensor and already hold the row sums, such as the NSA module:
 *   bwd_flags      0: as the entry point extended; otherwise a set of bits:
 *                  NSA_BWD_DQ_ACCUMULATE  this branch's dQ is added to the values dQ
 *                    already holds (same element type, added in fp32 and rounded
 *                    once), so no separate pass sums the branches' dQ;
 *                  NSA_BWD_DKDV_OVERWRITE  dK and dV are overwritten with this
 *                    branch's gradients (every element written, zeros where no query
 *                    sees a key) instead of added to, so the caller needs no zero
 *                    fill;
 *                  NSA_BWD_DQ_DEFER  (compression, for nsa_sliding_window_bwd_pair)
 *                    everything but the dQ kernel runs: dK / dV, and the stored dS and
 *                    re-packed K^T stay in the workspace for the paired call; needs
 *                    nsa_bwd_dq_deferrable() = 1 for the shape, else NSA_ERR_INVALID.
 *                  Other bits are rejected with NSA_ERR_INVALID.
 *   delta_in       null: as the entry point extended; otherwise the row sums
 *                  D = sum_d Out * dOut per (z, h, t) row, fp32, contiguous [Z, H, n_ctx_q],
 *                  which the backward then uses instead of reading Out.
 *   row_gate       null: as the entry point extended; otherwise a per-row gate
 *                  (fp32, contiguous [Z, H, n_ctx_q]): the branch's output gradient is
 *                  row_gate[z,h,t] * dOut (the gated mix of the NSA module,
 *                  nsa/kernels.py:2446-2463), so callers pass the mix's dOut unscaled.
 *   row_dot        null, or fp32 contiguous [Z, H, n_ctx_q] receiving sum_d dOut * Out
 *                  per row (the gradient of the row's gate); needs delta_in null.
 * With bwd_flags = 0 and the three pointers null each behaves exactly as the entry
 * point it extends. */
int nsa_sliding_window_bwd_ex(const void* Q, const void* K, const void* V, const void* Out, const void* dOut,
                           float sm_scale, const float* L, const float* M, int64_t stride_qz, int64_t stride_qh,
                           int64_t stride_qm, int64_t stride_qk, int64_t stride_kz, int64_t stride_kg,
                           int64_t stride_kn, int64_t stride_kk, int64_t stride_vz, int64_t stride_vg,
                           int64_t stride_vn, int64_t stride_vk, int64_t stride_oz, int64_t stride_oh,
                           int64_t stride_om, int64_t stride_ok, int64_t stride_lz, int64_t stride_lh,
                           int64_t stride_lm, int64_t stride_mz, int64_t stride_mh, int64_t stride_mm, void* dQ,
                           void* dK, void* dV, int64_t stride_dqz, int64_t stride_dqh, int64_t stride_dqm,
                           int64_t stride_dqk, int64_t stride_dkz, int64_t stride_dkg, int64_t stride_dkn,
                           int64_t stride_dkk, int64_t stride_dvz, int64_t stride_dvg, int64_t stride_dvn,
                           int64_t stride_dvk, int Z, int H, int n_kv_groups, int n_ctx, int window_size,
                           int head_dim_qk, int head_dim_v, int dtype,
                           int bwd_flags, const float* delta_in, const float* row_gate, float* row_dot, void* workspace, size_t workspace_bytes,
                           nsa_stream_t stream);

/* No counterpart in the reference (the NSA module's fused backward): the sliding-window
 * backward extension above, whose dQ kernel also adds the dQ of a compression backward
 * that ran before it (same stream) with NSA_BWD_DQ_DEFER over the same Q, dOut, sm_scale,
 * Z, H, n_kv_groups, n_ctx, head dims and dtype: cmp_block_ends / cmp_n_blocks are that
 * call's Block_ends / n_blocks and cmp_workspace its workspace (not reused in between).
 * Both branches' dQ are summed in fp32 and added to (NSA_BWD_DQ_ACCUMULATE) or written
 * over dQ once, so the running dQ is read and written once for the two.  Needs
 * nsa_bwd_dq_deferrable() = 1 for both shapes, else NSA_ERR_INVALID. */
int nsa_sliding_window_bwd_pair(const void* Q, const void* K, const void* V, const void* Out, const void* dOut,
                                float sm_scale, const float* L, const float* M, int64_t stride_qz,
                                int64_t stride_qh, int64_t stride_qm, int64_t stride_qk, int64_t stride_kz,
                                int64_t stride_kg, int64_t stride_kn, int64_t stride_kk, int64_t stride_vz,
                                int64_t stride_vg, int64_t stride_vn, int64_t stride_vk, int64_t stride_oz,
                                int64_t stride_oh, int64_t stride_om, int64_t stride_ok, int64_t stride_lz,
                                int64_t stride_lh, int64_t stride_lm, int64_t stride_mz, int64_t stride_mh,
                                int64_t stride_mm, void* dQ, void* dK, void* dV, int64_t stride_dqz,
                                int64_t stride_dqh, int64_t stride_dqm, int64_t stride_dqk, int64_t stride_dkz,
                                int64_t stride_dkg, int64_t stride_dkn, int64_t stride_dkk, int64_t stride_dvz,
                                int64_t stride_dvg, int64_t stride_dvn, int64_t stride_dvk, int Z, int H,
                                int n_kv_groups, int n_ctx, int window_size, int head_dim_qk, int head_dim_v,
                                int dtype, int bwd_flags, const float* delta_in, const float* row_gate,
                                float* row_dot, const int32_t* cmp_block_ends, int cmp_n_blocks,
                                const void* cmp_workspace, size_t cmp_workspace_bytes, void* workspace,
                                size_t workspace_bytes, nsa_stream_t stream);

int nsa_compression_bwd_ex(const void* Q, const void* K_blocks, const void* V_blocks, const int32_t* Block_ends,
                        const void* Out, const void* dOut, float sm_scale, const float* L, const float* M,
                        int64_t stride_qz, int64_t stride_qh, int64_t stride_qm, int64_t stride_qk,
                        int64_t stride_kz, int64_t stride_kg, int64_t stride_kn, int64_t stride_kk,
                        int64_t stride_vz, int64_t stride_vg, int64_t stride_vn, int64_t stride_vk,
                        int64_t stride_oz, int64_t stride_oh, int64_t stride_om, int64_t stride_ok,
                        int64_t stride_lz, int64_t stride_lh, int64_t stride_lm, int64_t stride_mz,
                        int64_t stride_mh, int64_t stride_mm, void* dQ, void* dK, void* dV, int64_t stride_dqz,
                        int64_t stride_dqh, int64_t stride_dqm, int64_t stride_dqk, int64_t stride_dkz,
                        int64_t stride_dkg, int64_t stride_dkn, int64_t stride_dkk, int64_t stride_dvz,
                        int64_t stride_dvg, int64_t stride_dvn, int64_t stride_dvk, int Z, int H, int n_kv_groups,
                        int n_ctx_q, int n_blocks, int head_dim_qk, int head_dim_v, int dtype,
                        int bwd_flags, const float* delta_in, const float* row_gate, float* row_dot, void* workspace,
                        size_t workspace_bytes, nsa_stream_t stream);

int nsa_sparse_selection_bwd_ex(const void* Q, const void* K, const void* V, const void* Block_indices, const void* Out,
                             const void* dOut, float sm_scale, const float* L, const float* M, int64_t stride_qz,
                             int64_t stride_qh, int64_t stride_qm, int64_t stride_qk, int64_t stride_kz,
                             int64_t stride_kg, int64_t stride_kn, int64_t stride_kk, int64_t stride_vz,
                             int64_t stride_vg, int64_t stride_vn, int64_t stride_vk, int64_t stride_oz,
                             int64_t stride_oh, int64_t stride_om, int64_t stride_ok, int64_t stride_bz,
                             int64_t stride_bg, int64_t stride_bm, int64_t stride_bn, int64_t stride_lz,
                             int64_t stride_lh, int64_t stride_lm, int64_t stride_mz, int64_t stride_mh,
                             int64_t stride_mm, void* dQ, void* dK, void* dV, int64_t stride_dqz, int64_t stride_dqh,
                             int64_t stride_dqm, int64_t stride_dqk, int64_t stride_dkz, int64_t stride_dkg,
                             int64_t stride_dkn, int64_t stride_dkk, int64_t stride_dvz, int64_t stride_dvg,
                             int64_t stride_dvn, int64_t stride_dvk, int Z, int H, int n_kv_groups, int n_ctx_q,
                             int n_ctx_kv, int n_slots, int block_size_selection, int is_causal, int index_is_int64,
                             int all_invalid_fallback, int head_dim_qk, int head_dim_v, int dtype,
                             int bwd_flags, const float* delta_in, const float* row_gate, float* row_dot, void* workspace,
                             size_t workspace_bytes, nsa_stream_t stream);


/* ---- kernel timing (no reference counterpart: profiling aid) ----------------
 * nsa_timing_begin(id) records a HIP event pair on the launch stream around every
 * subsequent launch of kernel `id` (0-2 forward of sliding/compression/selection,
 * 3-5 their dQ kernels, 6-8 their dK/dV kernels, 9 dK/dV partial reduce, 10 scoring
 * top-n, 11/12 compression pooling fwd/bwd); nsa_timing_end() waits for those events
 * and returns the summed milliseconds and the number of launches, then disarms. */
int nsa_timing_begin(int kernel_id);
int nsa_timing_end(double* total_ms, int* launches);

/* ---- allocation-free sliding-window forward ---------------------------------
 * No counterpart in the reference.  For callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc):
 * nsa_sliding_window_fwd with the same arguments and meaning, minus the workspace.  The
 * K/V re-pack goes to a static 32 MiB scratch array in the library (one copy per GPU,
 * held until the process ends); a shape whose nsa_fwd_workspace_size exceeds 32 MiB
 * returns NSA_ERR_WORKSPACE before anything is launched.  Nothing is allocated and no
 * allocating routine is called.  Every call on one GPU shares that GPU's scratch:
 * calls that overlap on one GPU (two streams, two threads) race; serialise them. */
int nsa_sliding_window_fwd_noalloc(const void* Q, const void* K, const void* V, void* Out, float sm_scale, float* L,
                                   float* M, int64_t stride_qz, int64_t stride_qh, int64_t stride_qm,
                                   int64_t stride_qk, int64_t stride_kz, int64_t stride_kg, int64_t stride_kn,
                                   int64_t stride_kk, int64_t stride_vz, int64_t stride_vg, int64_t stride_vn,
                                   int64_t stride_vk, int64_t stride_oz, int64_t stride_oh, int64_t stride_om,
                                   int64_t stride_ok, int64_t stride_lz, int64_t stride_lh, int64_t stride_lm,
                                   int64_t stride_mz, int64_t stride_mh, int64_t stride_mm, int Z, int H,
                                   int n_kv_groups, int n_ctx, int window_size, int head_dim_qk, int head_dim_v,
                                   int dtype, nsa_stream_t stream);

/* ---- dK/dV schedule query (no reference counterpart: introspection for tests) --
 * The number of dK/dV work items per (batch, KV group) and the query-segment length
 * (128 or 256 entries) the backward entry points launch with for this shape. */
int nsa_bwd_dkdv_plan(int branch, int Z, int H, int n_kv_groups, int n_ctx_q, int n_ctx_kv, int n_slots,
                      int block_size_selection, int window_size, int* items_per_bg, int* segment);

/* ---- selection scoring: Eq. 8 -> 9 -> 10 -> top-n, fused -------------------
 * Replaces the module's inline Eq. 8 (nsa/kernels.py:2316-2343),
 * derive_selection_from_compression_per_timestep (nsa/kernels.py:1920-1962) and
 * select_top_k_blocks_per_query_with_gqa (nsa/kernels.py:1965-2040).
 * q [Z,H,T,dk] and k_cmp [Z,G,dk,n_blocks] (element (z,g,e,i) at the given strides,
 * passed in (z, g, dk, block) order) share `dtype`; Block_ends int32 contiguous.
 * out_idx [Z,G,T,n] int64 (strides in elements).  p_cmp [Z,H,T,n_blocks] and
 * p_slc [Z,H,T,ceil(n_blocks/(l'/d))] are optional compact fp32 outputs (NULL to
 * skip).  fp32 arithmetic in a fixed order: indices are reproducible bit for bit.
 * include_fixed && n_fixed > 0 merges the blocks [0, max(0,(t-l')/l'), t/l'] first.
 * workspace: device memory, 16-byte aligned, of nsa_score_topn_workspace_size() bytes
 * (the fp32 logits of every row and block, then one int per 128-row logits tile);
 * NSA_ERR_WORKSPACE when smaller. */
size_t nsa_score_topn_workspace_size(int Z, int H, int n_kv_groups, int n_ctx, int head_dim_qk, int n_blocks, int n);
int nsa_score_topn(const void* q, const void* k_cmp, const int32_t* Block_ends, int64_t* out_idx, float* p_cmp,
                   float* p_slc, int64_t stride_qz, int64_t stride_qh, int64_t stride_qm, int64_t stride_qk,
                   int64_t stride_kz, int64_t stride_kg, int64_t stride_kk, int64_t stride_kn, int64_t stride_iz,
                   int64_t stride_ig, int64_t stride_im, int64_t stride_in, int Z, int H, int n_kv_groups, int n_ctx,
                   int head_dim_qk, int n_blocks, int l, int d, int l_prime, int n, int include_fixed, int n_fixed,
                   int dtype, float scale, void* workspace, size_t workspace_bytes, nsa_stream_t stream);

/* ---- gate activation and gated mix (NSAAttention.forward, nsa/kernels.py:2429-2463) --
 * No entry point of its own in the reference (torch elementwise ops there); fused here.
 * gate_act selects what the gate input z [B,H,T,3] (any strides) is: 0 the gates g
 * themselves; 1 logits, g = sigmoid(z); 2 logits, g = softmax over the three
 * (the reference's gate_mode "sigmoid" / "softmax", nsa/kernels.py:2436-2440).
 * Forward: out[b,h,t,:] = g0 o_cmp + g1 o_sel + g2 o_win, summed in fp32 and rounded once
 * (the reference's eval path sums in float64 and rounds once).  o_* share the strides
 * so_*, out any strides; every row unit-stride and 16-byte aligned.  Backward:
 * do_k = g_k dout (contiguous [B,H,T,dv]); dgates (contiguous fp32 [B,H,T,3]) is the
 * gradient of the gate input: dg_k = sum_d dout . o_k for gate_act 0, dg_k g_k (1 - g_k)
 * for 1, g_k (dg_k - sum_j g_j dg_j) for 2; delta, when not null, receives
 * delta[k][b,h,t] = g_k dg_k = sum_d o_k . do_k (contiguous fp32 [3,B,H,T]), the row
 * sums the branch backward extensions take as delta_in. */
int nsa_gate_mix_fwd(const void* o_cmp, const void* o_sel, const void* o_win, int64_t so_b, int64_t so_h,
                     int64_t so_t, const void* gates, int64_t sg_b, int64_t sg_h, int64_t sg_t, int64_t sg_k,
                     void* out, int64_t sout_b, int64_t sout_h, int64_t sout_t, int B, int H, int T, int dv,
                     int gate_act, int dtype, nsa_stream_t stream);
int nsa_gate_mix_bwd(const void* dout, int64_t sd_b, int64_t sd_h, int64_t sd_t, const void* o_cmp,
                     const void* o_sel, const void* o_win, int64_t so_b, int64_t so_h, int64_t so_t,
                     const void* gates, int64_t sg_b, int64_t sg_h, int64_t sg_t, int64_t sg_k, void* do_cmp,
                     void* do_sel, void* do_win, float* dgates, float* delta, int B, int H, int T, int dv,
                     int gate_act, int dtype, nsa_stream_t stream);

/* The gate activation alone, for the fused path whose mix runs in the sliding-window
 * forward's epilogue and whose branch backwards write the row dots (the reference
 * applies it inline, nsa/kernels.py:2436-2440).  gate_act as above.  Forward: gates
 * (contiguous fp32 [3,B,H,T]) = act(gate_in), gate_in [B,H,T,3] in dtype with strides
 * sz_*.  Backward: from the gates and row_dots r_k = sum_d dout . o_k (both contiguous
 * fp32 [3,B,H,T]), dgate_in (dtype, strides sz_*) receives the gradient of the gate
 * input: r_k (0), r_k g_k (1 - g_k) (1), g_k (r_k - sum_j g_j r_j) (2). */
int nsa_gate_act_fwd(const void* gate_in, int64_t sz_b, int64_t sz_h, int64_t sz_t, int64_t sz_k, float* gates, int B,
                     int H, int T, int gate_act, int dtype, nsa_stream_t stream);
int nsa_gate_act_bwd(const float* gates, const float* row_dots, void* dgate_in, int64_t sz_b, int64_t sz_h,
                     int64_t sz_t, int64_t sz_k, int B, int H, int T, int gate_act, int dtype, nsa_stream_t stream);

/* Row dots of the gated mix for the module backward (no reference counterpart: the
 * reference's autograd forms d out / d g_k = dout . o_k inside the mix backward,
 * nsa/kernels.py:2429-2463): dots[k][b][h][t] = sum_d dout[b,h,t,d] * o_k[b,h,t,d] for
 * k = 0 (o_cmp), 1 (o_sel), 2 (o_win), fp32 contiguous [3,B,H,T], dout read once.  They
 * feed nsa_gate_act_bwd as row_dots and each branch backward extension as delta_in, so
 * no branch backward reads its output.  dout and the o_k share the strides so_*, unit
 * feature stride, 16-byte aligned rows; dv 32, 64 or 128. */
int nsa_mix_row_dots(const void* dout, const void* o_cmp, const void* o_sel, const void* o_win, int64_t so_b,
                     int64_t so_h, int64_t so_t, float* dots, int B, int H, int T, int dv, int dtype,
                     nsa_stream_t stream);

/* ---- compression pooling (compress_tokens, nsa/kernels.py:2119-2208) --------
 * With the first MLP layer split as W1 = [W1k | W1p]:  Y = k W1k^T  [Z,G,T,width],
 * C = E W1p^T + b1  [l,width].  Forward writes R[i] = mean_{u<l} relu(Y[d*i+u] + C[u])
 * [Z,G,n_act,width] and V_cmp[i] = mean_{u<l} v[d*i+u] [Z,G,n_act,dv]; the caller
 * finishes K_cmp = R W2^T + b2.  Backward overwrites dY, dV (dtype) and dC (fp32).
 * All tensors compact row-major; with token_major set, Y / dY and V / dV are stored
 * [Z,T,G,*] (the layout of the module's K / V projections) instead of [Z,G,T,*]. */
int nsa_compress_pool_fwd(const void* Y, const void* C, const void* V, void* R, void* V_cmp, int Z, int n_kv_groups,
                          int n_ctx, int width, int head_dim_v, int l, int d, int n_act, int token_major, int dtype,
                          nsa_stream_t stream);
int nsa_compress_pool_bwd(const void* Y, const void* C, const void* dR, const void* dV_cmp, void* dY, float* dC,
                          void* dV, int Z, int n_kv_groups, int n_ctx, int width, int head_dim_v, int l, int d,
                          int n_act, int token_major, int dtype, nsa_stream_t stream);

/* ---- weight gradient of the compression MLP's token-wise layers ----------------------
 * No counterpart in the reference (autograd computes it there).  dW [n1, n2] (leading
 * dimension ld_dw) = dY^T X over `rows` token rows: dY [rows, n1], X [rows, n2], bf16,
 * unit feature stride, 16-byte aligned rows (leading dimensions ld_dy, ld_x multiples of
 * 8); n1, n2 multiples of 64.  The rows are summed in fixed chunks on the matrix cores in
 * fp32 and the chunks added in order (reproducible), rounded to bf16 once.  workspace:
 * nsa_wgrad_workspace_size(rows, n1, n2) bytes (fp32 partial tiles).  Other dtypes:
 * NSA_ERR_UNSUPPORTED. */
size_t nsa_wgrad_workspace_size(int rows, int n1, int n2);
int nsa_wgrad(const void* dY, int64_t ld_dy, const void* X, int64_t ld_x, int rows, int n1, int n2, void* dW,
              int64_t ld_dw, int dtype, void* workspace, size_t workspace_bytes, nsa_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* NSA_HIP_H */
