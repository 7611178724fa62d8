// Shared argument blocks and launch helpers for the NSA attention kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nsa {

enum Branch : int { kSliding = 0, kCompression = 1, kSelection = 2 };
enum DType : int { kF32 = 0, kBF16 = 1 };

// Columns handled by one dense forward workgroup (kFwdWaves waves x NSUB x 16) and one
// dense dQ workgroup (kDqWaves waves x 16).
constexpr int kFwdNSub = 1;
constexpr int kFwdWaves = 8;
constexpr int kFwdCols = kFwdWaves * kFwdNSub * 16;
constexpr int kDqWaves = 12;
constexpr int kDqNSub = 1;
constexpr int kDqCols = kDqWaves * kDqNSub * 16;
// Distinct selection blocks a row's union bitmap can hold.
constexpr int kSelMaxBlocks = 4096;
// Query rows staged per step of the dK/dV kernels.
constexpr int kRowChunk = 32;
// Compression dQ from the stored dS keeps the block end of every 32-key chunk's first key
// in LDS; the host stores dS for compression only up to this many chunks (65536 blocks).
constexpr int kDqCbeMax = 2048;
// Query entries (timesteps; selection: CSR entries) per dK/dV work item: 128 or 256,
// chosen per launch (dkdv_seg_len), at most kSegTMax.
constexpr int kSegTMax = 256;
// dK/dV key tiles (all batches and groups) from which the sliding-window backward gives
// each tile all its query rows in one work item (one item per CU or more)
constexpr int kDkdvDirectItems = 256;

// Dynamic LDS above the 64 KB a kernel may use by default needs the kernel's limit
// raised first; smaller launches skip that runtime call.
inline void allow_dynamic_lds(const void* fn, size_t bytes) {
  if (bytes > 64 * 1024) (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

struct AttnArgs {
  // queries [B,H,Tq,DK], unit stride on the feature axis
  const void* q;
  int64_t sq_b, sq_h, sq_t;
  // group K/V re-packed by the prep kernel (Tp rows, zero padded) in fragment-native
  // layouts: every 16-byte MFMA fragment of a wave is one contiguous 1 KB run
  //   krf K rowfrag, kcf K colfrag (K^T), vrf V rowfrag, vcf V colfrag (V^T)
  const void* krf;
  const void* kcf;
  const void* vrf;
  const void* vcf;
  int Tp;
  // forward outputs / backward inputs
  void* o;
  int64_t so_b, so_h, so_t;
  float* L;
  int64_t sl_b, sl_h, sl_t;
  float* M;
  int64_t sm_b, sm_h, sm_t;
  // backward
  const void* dout;
  int64_t sdo_b, sdo_h, sdo_t;
  void* dq;
  int64_t sdq_b, sdq_h, sdq_t;
  int dq_acc;  // 1: dQ is added to the destination's values instead of overwriting them
  const float* delta_in;  // null, or the caller's rowsum(O*dO) [B,H,Tq] compact (O is then not read)
  // gated mix (the NSA module): this branch's output gradient is row_gate[row] * dOut
  const float* row_gate;  // [B,H,Tq] compact fp32 activated gate of this branch, or null (1)
  float* row_dot;         // [B,H,Tq] compact fp32: receives sum_d dOut * Out per row, or null
  // forward mix epilogue (sliding / compression kernel): mix_out = g0 mix_o0 + g1 mix_o1 + g2 Out
  void* mix_out;
  int64_t smx_b, smx_h, smx_t;
  const void* mix_o0;  // the other two branch outputs, with Out's strides
  const void* mix_o1;
  const float* mix_gates;  // [3,B,H,Tq] compact fp32 activated gates (0, 1: mix_o0 / mix_o1, 2: Out)
  // per query row, for the dK/dV kernels: {lse2 = (M+L)*log2(e) (+inf for empty rows),
  // delta = rowsum(O*dO), gate (1 without a row gate), 0}, in [B*G][Tq][hpg] order so the
  // heads of one timestep share cache lines
  float4* rstat;
  // dK/dV destination (accumulated into, or overwritten with dkdv_ow; any strides) or fp32 partials
  void* dk;
  int64_t sdk_b, sdk_g, sdk_t, sdk_d;
  void* dv;
  int64_t sdv_b, sdv_g, sdv_t, sdv_d;
  void* partial;  // [items][keys][DK+DV] partial sums, fp32 (bf16 for bf16 inputs)
  int items_per_bg;
  int q0;  // absolute position of query row 0 (0 unless a caller decodes past a cache)
  int seg;  // query entries per dK/dV work item
  int direct;  // dK/dV items accumulate into dk / dv themselves (one item per key tile)
  int dkdv_ow;  // 1: dK / dV are overwritten (every element written) instead of added to
  // shapes
  int B, H, G, hpg, Tq, Tkv;
  float scale;
  // branch parameters
  int window;
  const int* block_ends;  // [Tkv] int32 (compression)
  const int* sel;         // cleaned selection [B,G,Tq,nslots] int32, ascending, -1 padded
  int nslots;
  int lprime;
  int nblk;               // ceil(Tkv / lprime)
  int causal;             // selection: mask keys after the query position
  // selection CSR (backward)
  const int* csr_off;     // [B,G,nblk+1]
  const int* csr_t;       // [B,G,Tq*nslots] query timesteps per block, ascending
  const int* seg_off;     // [B,G,nblk+1] work-item prefix per block
  const int* csr_s;       // [B,G,Tq*nslots] the slot of each CSR entry in its timestep's cleaned list
  // selection, stored-dS backward (bf16, hpg and l' multiples of 16 and 64): the dK/dV
  // kernel writes every (timestep, slot) pair's dS in the MFMA operand order of the dQ
  // product, and the dQ kernel reads it instead of recomputing S and dP:
  //   ds[b,g][t][slot][64-key sub-block][16-head group] = 2 fragments x 64 lanes x 8 bf16
  // and the same for the sliding-window / compression backward, per 32-key chunk:
  //   ds[b,g][t][16-head group][ds_nch chunks from the timestep's first visible one]
  //   = 64 lanes x 8 bf16 (sliding: chunks from max(0, t - window + 1) / 32; compression:
  //   from chunk 0)
  void* ds;
  int ds_nch;
  // sliding-window dQ from the stored dS only: a compression backward over the same
  // queries whose dQ is added in the same pass (its K^T colfrags, stored dS, block ends,
  // compressed length, re-packed rows and dS chunks per timestep; pair_ds null: none)
  const void* pair_kcf;
  const void* pair_ds;
  const int* pair_block_ends;
  int pair_Tkv, pair_Tp, pair_ds_nch;
};

template <typename T, int DK, int DV, int BR>
void launch_attn_fwd(const AttnArgs& a, hipStream_t s);
template <typename T, int DK, int DV, int BR>
void launch_attn_bwd_dq(const AttnArgs& a, hipStream_t s);
template <typename T, int DK, int DV, int BR>
void launch_attn_bwd_dkdv(const AttnArgs& a, hipStream_t s);

}  // namespace nsa
