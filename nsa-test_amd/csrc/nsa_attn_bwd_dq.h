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
  static_assert(BR == kSliding || BR == kCompression, "selection uses attn_sel_dq_kernel");
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
  // bf16 reads the K^T operand from the K rows with the LDS transpose load; fp32 stages
  // a K^T copy from the kn layout
  constexpr bool kTr = sizeof(S) == 2;
  static_assert(DK % KC == 0 && DV % KC == 0, "head dims");

  __shared__ __attribute__((aligned(16))) S Ks[64 * KP];                 // K rows   [key][d]
  __shared__ __attribute__((aligned(16))) S KnS[kTr ? 8 : DK * NP];      // K^T      [d][key]
  __shared__ __attribute__((aligned(16))) S Vns[64 * VP];                // V rows   [key][dv]
  __shared__ int s_be[64];
  __shared__ int s_misc[4];

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
  // sliding: the column sees keys [kmin_s, kmin_s + kspan_s) (branch-free test)
  const int kmin_s = max(colt - a.window + 1, 0);
  const uint32_t kspan_s = colv ? (uint32_t)max(0, min(colt, a.Tkv - 1) + 1 - kmin_s) : 0u;

  f32x4 dqa[DK / 16];
#pragma unroll
  for (int j = 0; j < DK / 16; ++j) dqa[j] = zero4();

  int ntiles = 0, key_lo = 0;
  if (BR == kSliding) {
    key_lo = max(0, t_first - a.window + 1) & ~31;  // 32-key aligned (C-permuted K^T chunks)
    const int hi = min(t_last, a.Tkv - 1);
    ntiles = hi >= key_lo ? (hi - key_lo) / 64 + 1 : 0;
  } else {
    if (tid == 0) s_misc[0] = 0;
    __syncthreads();
    int mx = 0;
    for (int i = tid; i < a.Tkv; i += 256)
      if (a.block_ends[i] <= t_last) mx = i + 1;
    if (mx) atomicMax(&s_misc[0], mx);
    __syncthreads();
    ntiles = (s_misc[0] + 63) / 64;
  }

  // ---- tile operands, loaded into registers one tile ahead ----
  constexpr int NKP = (64 * (DK / EPF) + 255) / 256;
  constexpr int NNP = kTr ? 1 : (DK * (64 / EPF) + 255) / 256;
  constexpr int NVP = (64 * (DV / EPF) + 255) / 256;
  u32x4 pk[NKP], pn[NNP], pv[NVP];
  int pbe = 0x7fffffff;
  auto tile_key0 = [&](int it) -> int { return BR == kSliding ? key_lo + it * 64 : it * 64; };
  auto load_tile = [&](int key0) {
#pragma unroll
    for (int j = 0; j < NKP; ++j) {
      const int c = min(tid + 256 * j, 64 * (DK / EPF) - 1);
      pk[j] = *reinterpret_cast<const u32x4*>(kt + (int64_t)(key0 + c / (DK / EPF)) * DK + (c % (DK / EPF)) * EPF);
    }
    if constexpr (!kTr) {
#pragma unroll
      for (int j = 0; j < NNP; ++j) {
        const int c = min(tid + 256 * j, DK * (64 / EPF) - 1);
        pn[j] = *reinterpret_cast<const u32x4*>(kn + (int64_t)(c / (64 / EPF)) * a.Tp + key0 + (c % (64 / EPF)) * EPF);
      }
    }
#pragma unroll
    for (int j = 0; j < NVP; ++j) {
      const int c = min(tid + 256 * j, 64 * (DV / EPF) - 1);
      pv[j] = *reinterpret_cast<const u32x4*>(vn + (int64_t)(key0 + c / (DV / EPF)) * DV + (c % (DV / EPF)) * EPF);
    }
    if (BR == kCompression && tid < 64) {
      const int key = key0 + tid;
      pbe = key < a.Tkv ? a.block_ends[key] : 0x7fffffff;
    }
  };
  if (ntiles > 0) load_tile(tile_key0(0));

  for (int it = 0; it < ntiles; ++it) {
    const int key0 = tile_key0(it);
#pragma unroll
    for (int j = 0; j < NKP; ++j) {
      const int c = tid + 256 * j;
      if ((64 * (DK / EPF)) % 256 == 0 || c < 64 * (DK / EPF))
        *reinterpret_cast<u32x4*>(&Ks[(c / (DK / EPF)) * KP + (c % (DK / EPF)) * EPF]) = pk[j];
    }
    if constexpr (!kTr) {
#pragma unroll
      for (int j = 0; j < NNP; ++j) {
        const int c = tid + 256 * j;
        if ((DK * (64 / EPF)) % 256 == 0 || c < DK * (64 / EPF))
          *reinterpret_cast<u32x4*>(&KnS[(c / (64 / EPF)) * NP + (c % (64 / EPF)) * EPF]) = pn[j];
      }
    }
#pragma unroll
    for (int j = 0; j < NVP; ++j) {
      const int c = tid + 256 * j;
      if ((64 * (DV / EPF)) % 256 == 0 || c < 64 * (DV / EPF))
        *reinterpret_cast<u32x4*>(&Vns[(c / (DV / EPF)) * VP + (c % (DV / EPF)) * EPF]) = pv[j];
    }
    if (BR == kCompression && tid < 64) s_be[tid] = pbe;
    __syncthreads();
    if (it + 1 < ntiles) load_tile(tile_key0(it + 1));

    int be_max = 0;
    if (BR == kCompression) {
      be_max = s_be[lane];
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) be_max = max(be_max, __shfl_xor(be_max, o));
    }

    // Every (subtile, tile) pair runs the products, fully masked when no key is
    // visible: a branch around them would make the compiler move the accumulators
    // between register files on every tile.
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
    else
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
          if (BR == kSliding) ok = (uint32_t)(key - kmin_s) < kspan_s;
          else ok = colv & (s_be[ks * 16 + 4 * g4 + i] <= colt);
          p = ok ? fast_exp2(st[ks][i] * scale2 - l2) : 0.f;
        }
        st[ks][i] = p * (dp[ks][i] - dl);  // dS^T
      }
    }
#pragma unroll
    for (int kc2 = 0; kc2 < 64 / CK; ++kc2) {
      const uint4 sf = CFrag<T>::pack(st[kc2 * CT], st[kc2 * CT + CT - 1]);
      if constexpr (kTr) {
        // A = K^T (16 features x the 32 keys of the C-permuted CFrag order) from the
        // K rows: lanes 4*rho+q of group g4 address key kc2*32 + 4*g4 + rho (then +16)
        const int r0 = kc2 * CK + 4 * g4 + (c16 >> 2);
        const int f4 = 4 * (c16 & 3);
#pragma unroll
        for (int j = 0; j < DK / 16; ++j)
          dqa[j] = Mma<T>::run(dqa[j], ld_tr_pair(&Ks[r0 * KP + j * 16 + f4], 16 * KP), sf);
      } else {
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
