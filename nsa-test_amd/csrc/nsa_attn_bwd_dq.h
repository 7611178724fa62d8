// Backward attention for the three NSA branches on gfx950, split FlashAttention-2
// style into a query-major dQ kernel and a key-major dK/dV kernel.  Neither uses
// floating-point atomics: each dQ row and each dK/dV row has exactly one owner, and
// where one key tile's queries are spread over several work items (compression,
// selection) the items write fp32 partials that a reduce kernel sums in a fixed
// order.  Results are therefore bit-reproducible run to run.
//
// Math (reference backward, nsa/kernels.py:1303-1530): with s = scale * q.k,
//   p  = exp(s - M - L)                    (saved forward statistics)
//   dP = dO . v,   D = rowsum(O * dO),   dS = p * (dP - D)
//   dQ = scale * dS . K      dK = scale * dS^T . Q      dV = p^T . dO
#pragma once
#include "nsa_attn.h"
#include "nsa_device.h"
#include "nsa_attn_sel.h"

namespace nsa {

// ============================== dQ (query-major) ===============================
template <typename T, int DK, int DV, int BR>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(AttnArgs a) {
  using S = typename Store<T>::type;
  constexpr int EPF = Elem<T>::kPerFrag;
  constexpr int KC = Elem<T>::kKChunk;
  constexpr int NKC = DK / KC;
  constexpr int NVC = DV / KC;
  constexpr int KP = DK + EPF;
  constexpr int NP = 64 + EPF;
  constexpr int VP = DV + EPF;
  constexpr int CK = CFrag<T>::kKeys;
  constexpr int CT = CK / 16;
  static_assert(DK % KC == 0 && DV % KC == 0, "head dims");

  __shared__ __attribute__((aligned(16))) S Ks[64 * KP];   // K rows   [key][d]
  __shared__ __attribute__((aligned(16))) S KnS[DK * NP];  // K^T      [d][key]
  __shared__ __attribute__((aligned(16))) S Vns[64 * VP];  // V rows   [key][dv]
  __shared__ int s_be[64];
  __shared__ int s_misc[4];
  __shared__ int s_list[BR == kSelection ? kSelListMax : 1];
  __shared__ int s_union[BR == kSelection ? kSelMaxBlocks : 1];
  __shared__ uint32_t s_bits[BR == kSelection ? kSelMaxBlocks / 32 : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g4 = lane >> 4;
  const int c16 = lane & 15;
  const int bg = blockIdx.y;
  const int b = bg / a.G;
  const int grp = bg % a.G;
  const int hpg = a.hpg;
  const int ncols = a.Tq * hpg;
  const int col_base = blockIdx.x * kDqCols;
  const int t_first = col_base / hpg;
  const int t_last = min(a.Tq - 1, (col_base + kDqCols - 1) / hpg);
  const float scale2 = a.scale * kLog2e;

  const S* kt = reinterpret_cast<const S*>(a.kt) + (int64_t)bg * a.Tp * DK;
  const S* kn = reinterpret_cast<const S*>(a.kn) + (int64_t)bg * DK * a.Tp;
  const S* vn = reinterpret_cast<const S*>(a.vn) + (int64_t)bg * a.Tp * DV;

  // one 16-column subtile per wave
  const int f0 = col_base + wave * 16;
  const int f = f0 + c16;
  const bool colv = f < ncols;
  const int colt = colv ? f / hpg : 0;
  const int colh = colv ? grp * hpg + f % hpg : 0;
  const int sub_t0 = f0 / hpg;
  const int sub_t1 = f0 < ncols ? min(a.Tq - 1, (f0 + 15) / hpg) : -1;
  uint4 qf[NKC], dof[NVC];
  {
    const S* qp = reinterpret_cast<const S*>(a.q) + b * a.sq_b + (int64_t)colh * a.sq_h + (int64_t)colt * a.sq_t;
    const S* dp = reinterpret_cast<const S*>(a.dout) + b * a.sdo_b + (int64_t)colh * a.sdo_h +
                  (int64_t)colt * a.sdo_t;
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc)
      qf[kc] = colv ? *reinterpret_cast<const uint4*>(qp + kc * KC + g4 * EPF) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int kc = 0; kc < NVC; ++kc)
      dof[kc] = colv ? *reinterpret_cast<const uint4*>(dp + kc * KC + g4 * EPF) : make_uint4(0, 0, 0, 0);
  }
  const int64_t srow = ((int64_t)b * a.H + colh) * a.Tq + colt;
  const float l2 = colv ? a.lse2[srow] : INFINITY;
  const float dl = colv ? a.delta[srow] : 0.f;

  f32x4 dqa[DK / 16];
#pragma unroll
  for (int j = 0; j < DK / 16; ++j) dqa[j] = zero4();

  int ntiles = 0, key_lo = 0, nsubblk = 1;
  if (BR == kSliding) {
    key_lo = max(0, t_first - a.window + 1) & ~31;  // 32-key aligned (C-permuted K^T chunks)
    const int hi = min(t_last, a.Tkv - 1);
    ntiles = hi >= key_lo ? (hi - key_lo) / 64 + 1 : 0;
  } else if (BR == kCompression) {
    if (tid == 0) s_misc[0] = 0;
    __syncthreads();
    int mx = 0;
    for (int i = tid; i < a.Tkv; i += 256)
      if (a.block_ends[i] <= t_last) mx = i + 1;
    if (mx) atomicMax(&s_misc[0], mx);
    __syncthreads();
    ntiles = (s_misc[0] + 63) / 64;
  } else {
    const int nt = t_last - t_first + 1;
    const int total = nt * a.nslots;
    const int nwords = (a.nblk + 31) / 32;
    for (int i = tid; i < nwords; i += 256) s_bits[i] = 0;
    __syncthreads();
    const int* selrow = a.sel + ((int64_t)bg * a.Tq + t_first) * a.nslots;
    for (int i = tid; i < total; i += 256) {
      const int v = selrow[i];
      s_list[i] = v;
      if (v >= 0) atomicOr(&s_bits[v >> 5], 1u << (v & 31));
    }
    __syncthreads();
    if (tid == 0) {
      int n = 0;
      for (int w = 0; w < nwords; ++w) {
        uint32_t bits = s_bits[w];
        while (bits) {
          const int bit = __builtin_ctz(bits);
          bits &= bits - 1;
          s_union[n++] = w * 32 + bit;
        }
      }
      s_misc[0] = n;
    }
    __syncthreads();
    nsubblk = (a.lprime + 63) / 64;
    ntiles = s_misc[0] * nsubblk;
  }

  for (int it = 0; it < ntiles; ++it) {
    int key0, blk_lo = 0, blk_hi = 0;
    if (BR == kSliding) {
      key0 = key_lo + it * 64;
    } else if (BR == kCompression) {
      key0 = it * 64;
    } else {
      const int blk = s_union[it / nsubblk];
      blk_lo = blk * a.lprime;
      blk_hi = min(blk_lo + a.lprime, a.Tkv);
      key0 = blk_lo + (it % nsubblk) * 64;
      if ((a.causal && key0 > t_last) || key0 >= blk_hi) continue;
    }
    for (int c = tid; c < 64 * (DK / EPF); c += 256) {
      const int r = c / (DK / EPF);
      const int e = (c % (DK / EPF)) * EPF;
      *reinterpret_cast<uint4*>(&Ks[r * KP + e]) = *reinterpret_cast<const uint4*>(kt + (int64_t)(key0 + r) * DK + e);
    }
    for (int c = tid; c < DK * (64 / EPF); c += 256) {
      const int r = c / (64 / EPF);
      const int e = (c % (64 / EPF)) * EPF;
      *reinterpret_cast<uint4*>(&KnS[r * NP + e]) = *reinterpret_cast<const uint4*>(kn + (int64_t)r * a.Tp + key0 + e);
    }
    for (int c = tid; c < 64 * (DV / EPF); c += 256) {
      const int r = c / (DV / EPF);
      const int e = (c % (DV / EPF)) * EPF;
      *reinterpret_cast<uint4*>(&Vns[r * VP + e]) = *reinterpret_cast<const uint4*>(vn + (int64_t)(key0 + r) * DV + e);
    }
    if (BR == kCompression && tid < 64) {
      const int key = key0 + tid;
      s_be[tid] = key < a.Tkv ? a.block_ends[key] : 0x7fffffff;
    }
    __syncthreads();

    bool active;
    bool colsel = false;
    int be_max = 0;
    if (BR == kSliding) {
      active = sub_t1 >= 0 && key0 <= sub_t1 && key0 + 63 > sub_t0 - a.window;
    } else if (BR == kCompression) {
      int be_min = s_be[lane];
      be_max = be_min;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        be_min = min(be_min, __shfl_xor(be_min, o));
        be_max = max(be_max, __shfl_xor(be_max, o));
      }
      active = sub_t1 >= 0 && be_min <= sub_t1;
    } else {
      if (colv && (!a.causal || key0 <= colt)) {
        const int* lst = &s_list[(colt - t_first) * a.nslots];
        const int blk = blk_lo / a.lprime;
        for (int j = 0; j < a.nslots; ++j) {
          const int v = lst[j];
          if (v == blk) colsel = true;
          if (v < 0 || v >= blk) break;
        }
      }
      active = __ballot(colsel) != 0ull;
    }

    if (active) {
      f32x4 st[4], dp[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        st[ks] = zero4();
        dp[ks] = zero4();
        const S* krow = &Ks[(ks * 16 + c16) * KP];
        const S* vrow = &Vns[(ks * 16 + c16) * VP];
#pragma unroll
        for (int kc = 0; kc < NKC; ++kc) st[ks] = Mma<T>::run(st[ks], frag_std<T>(krow + kc * KC, g4), qf[kc]);
#pragma unroll
        for (int kc = 0; kc < NVC; ++kc) dp[ks] = Mma<T>::run(dp[ks], frag_std<T>(vrow + kc * KC, g4), dof[kc]);
      }
      bool all_visible = false;
      const bool full = f0 + 16 <= ncols;
      if (BR == kSliding)
        all_visible = full && key0 + 63 <= sub_t0 && key0 > sub_t1 - a.window && key0 + 63 < a.Tkv;
      else if (BR == kCompression)
        all_visible = full && be_max <= sub_t0;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float p;
          if (all_visible) {
            p = fast_exp2(st[ks][i] * scale2 - l2);
          } else {
            const int key = key0 + ks * 16 + 4 * g4 + i;
            bool ok;
            if (BR == kSliding) {
              ok = colv && key <= colt && key > colt - a.window && key < a.Tkv;
            } else if (BR == kCompression) {
              ok = colv && s_be[ks * 16 + 4 * g4 + i] <= colt;
            } else {
              ok = colsel && (!a.causal || key <= colt) && key < blk_hi;
            }
            p = ok ? fast_exp2(st[ks][i] * scale2 - l2) : 0.f;
          }
          st[ks][i] = p * (dp[ks][i] - dl);  // dS^T
        }
      }
#pragma unroll
      for (int kc2 = 0; kc2 < 64 / CK; ++kc2) {
        const uint4 sf = CFrag<T>::pack(st[kc2 * CT], st[kc2 * CT + CT - 1]);
#pragma unroll
        for (int j = 0; j < DK / 16; ++j) {
          const uint4 kf = frag_cperm<T>(&KnS[(j * 16 + c16) * NP + kc2 * CK], g4);
          dqa[j] = Mma<T>::run(dqa[j], kf, sf);
        }
      }
    }
    __syncthreads();
  }

  if (colv) {
    S* dqp = reinterpret_cast<S*>(a.dq) + b * a.sdq_b + (int64_t)colh * a.sdq_h + (int64_t)colt * a.sdq_t;
#pragma unroll
    for (int j = 0; j < DK / 16; ++j) store4<T>(dqp + j * 16 + 4 * g4, dqa[j] * a.scale);
  }
}

template <typename T, int DK, int DV, int BR>
void launch_attn_bwd_dq(const AttnArgs& a, hipStream_t s) {
  dim3 grid((a.Tq * a.hpg + kDqCols - 1) / kDqCols, a.B * a.G);
  if constexpr (BR == kSelection) {
    launch_attn_sel_dq<T, DK, DV>(a, s);  // per-wave selection kernel
  } else {
    hipLaunchKernelGGL((attn_bwd_dq_kernel<T, DK, DV, BR>), grid, dim3(256), 0, s, a);
  }
}

}  // namespace nsa
