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
// Workgroup = kDqWaves waves x 16 query columns.  The operands of a 64-key tile --
// K rowfrags (S^T = K Q^T), V rowfrags (dP^T = V dO^T) and K^T colfrags
// (dQ^T += K^T dS^T) -- are copied global -> LDS by direct-to-LDS loads from the
// fragment-native krf / vrf / kcf layouts, one 1 KB MFMA fragment per instruction, into a
// double buffer when two fit 136 KB (one workgroup of 12 waves per CU, three waves per SIMD),
// and every fragment read is a conflict-free 16-byte-per-lane LDS read.
template <typename T, int DK, int DV>
struct DqTile {
  static constexpr int KC = Elem<T>::kKChunk;
  static constexpr int CK = CFrag<T>::kKeys;
  static constexpr int NKF = 4 * (DK / KC);           // K rowfrags (ks, kc)
  static constexpr int NVF = 4 * (DV / KC);           // V rowfrags (ks, kc)
  static constexpr int NTF = (64 / CK) * (DK / 16);   // K^T colfrags (kc2, j)
  static constexpr int NF = NKF + NVF + NTF;
  static constexpr int BYTES = NF * 1024;
  static constexpr int NBUF = 2 * BYTES <= 136 * 1024 ? 2 : 1;
};

template <typename T, int DK, int DV, int BR>
__global__ __launch_bounds__(64 * kDqWaves) void attn_bwd_dq_kernel(AttnArgs a) {
  static_assert(BR == kSliding || BR == kCompression, "selection uses attn_sel_dq_kernel");
  using S = typename Store<T>::type;
  using TL = DqTile<T, DK, DV>;
  constexpr int EPF = Elem<T>::kPerFrag;
  constexpr int KC = Elem<T>::kKChunk;
  constexpr int NKC = DK / KC;
  constexpr int NVC = DV / KC;
  constexpr int CK = CFrag<T>::kKeys;
  constexpr int CT = CK / 16;
  constexpr int NW = kDqWaves;
  static_assert(DK % KC == 0 && DV % KC == 0, "head dims");

  extern __shared__ __attribute__((aligned(16))) uint4 dq_lds[];  // [NBUF][NF][64]
  __shared__ int s_be[2][64];
  __shared__ int s_misc[4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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

  const S* krf = reinterpret_cast<const S*>(a.krf) + (int64_t)bg * a.Tp * DK;
  const S* kcf = reinterpret_cast<const S*>(a.kcf) + (int64_t)bg * DK * a.Tp;
  const S* vrf = reinterpret_cast<const S*>(a.vrf) + (int64_t)bg * a.Tp * DV;

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
    for (int i = tid; i < a.Tkv; i += blockDim.x)
      if (a.block_ends[i] <= t_last) mx = i + 1;
    if (mx) atomicMax(&s_misc[0], mx);
    __syncthreads();
    ntiles = (s_misc[0] + 63) / 64;
  }

  // ---- the direct-to-LDS copy of one tile: wave w copies fragments w, w + NW, ... ----
  auto copy_tile = [&](int key0, int buf) __attribute__((always_inline)) {
    uint4* dst = dq_lds + buf * TL::NF * 64;
    for (int fr = wave; fr < TL::NF; fr += NW) {
      const S* src;
      if (fr < TL::NKF) {  // K rowfrag (16-key group (key0 >> 4) + ks, feature chunk kc)
        const int ks = fr / NKC, kc = fr % NKC;
        src = krf + ((((int64_t)(key0 >> 4) + ks) * NKC + kc) * 64 + lane) * EPF;
      } else if (fr < TL::NKF + TL::NVF) {  // V rowfrag
        const int v = fr - TL::NKF, ks = v / NVC, kc = v % NVC;
        src = vrf + ((((int64_t)(key0 >> 4) + ks) * NVC + kc) * 64 + lane) * EPF;
      } else {  // K^T colfrag (key chunk key0 / CK + kc2, feature group j)
        const int v = fr - TL::NKF - TL::NVF, kc2 = v / (DK / 16), j = v % (DK / 16);
        src = kcf + ((((int64_t)(key0 / CK) + kc2) * (DK / 16) + j) * 64 + lane) * EPF;
      }
      copy16_to_lds(src, dst + fr * 64);
    }
  };
  auto tile_key0 = [&](int it) -> int { return BR == kSliding ? key_lo + it * 64 : it * 64; };
  int pbe = 0x7fffffff;
  auto load_be = [&](int key0) {
    if (BR == kCompression && tid < 64) {
      const int key = key0 + tid;
      pbe = key < a.Tkv ? a.block_ends[key] : 0x7fffffff;
    }
  };
  if (ntiles > 0) {
    copy_tile(tile_key0(0), 0);
    load_be(tile_key0(0));
  }
  // row statistics after the first tile's copies are issued (their O loads overlap them)
  float l2, dl, rgate;
  dq_row_stats<T, NVC>(a, b, colh, colt, colv, dof, g4, srow, l2, dl, rgate);

  for (int it = 0; it < ntiles; ++it) {
    const int key0 = tile_key0(it);
    const int buf = TL::NBUF == 2 ? (it & 1) : 0;
    if (BR == kCompression && tid < 64) s_be[it & 1][tid] = pbe;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's copies of tile it have landed
    __syncthreads();                // every wave's have; tile it-1 is no longer read
    if (TL::NBUF == 2 && it + 1 < ntiles) {
      copy_tile(tile_key0(it + 1), buf ^ 1);
      load_be(tile_key0(it + 1));
    }
    const uint4* kb = dq_lds + buf * TL::NF * 64;
    const uint4* vb = kb + TL::NKF * 64;
    const uint4* tb = vb + TL::NVF * 64;
    const int* sbe = s_be[it & 1];

    int be_max = 0;
    if (BR == kCompression) {
      be_max = wave_butterfly(sbe[lane], [](int x, int y) { return max(x, y); });
    }

    // Every (subtile, tile) pair runs the products, fully masked when no key is
    // visible: a branch around them would make the compiler move the accumulators
    // between register files on every tile.
    f32x4 st[4], dp[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      st[ks] = zero4();
      dp[ks] = zero4();
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc) st[ks] = Mma<T>::run(st[ks], kb[(ks * NKC + kc) * 64 + lane], qf[kc]);
#pragma unroll
      for (int kc = 0; kc < NVC; ++kc) dp[ks] = Mma<T>::run(dp[ks], vb[(ks * NVC + kc) * 64 + lane], dof[kc]);
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
        bool ok = true;
        if (!all_visible) {
          const int key = key0 + ks * 16 + 4 * g4 + i;
          if (BR == kSliding) ok = (uint32_t)(key - kmin_s) < kspan_s;
          else ok = colv & (sbe[ks * 16 + 4 * g4 + i] <= colt);
        }
        // the mask on the exponent argument: no divergent branch around the exp
        const float p = fast_exp2(ok ? st[ks][i] * scale2 - l2 : -INFINITY);
        st[ks][i] = p * (dp[ks][i] - dl);  // dS^T
      }
    }
#pragma unroll
    for (int kc2 = 0; kc2 < 64 / CK; ++kc2) {
      const uint4 sf = CFrag<T>::pack(st[kc2 * CT], st[kc2 * CT + CT - 1]);
#pragma unroll
      for (int j = 0; j < DK / 16; ++j) dqa[j] = Mma<T>::run(dqa[j], tb[(kc2 * (DK / 16) + j) * 64 + lane], sf);
    }
    if (TL::NBUF == 1 && it + 1 < ntiles) {  // single buffer: refill once every wave is done
      __syncthreads();
      copy_tile(tile_key0(it + 1), 0);
      load_be(tile_key0(it + 1));
    }
  }

  if (colv) {
    // accumulate mode: the caller's running dQ (loaded here, not at the start: the
    // registers are not spare in this kernel)
    S* dqp = reinterpret_cast<S*>(a.dq) + b * a.sdq_b + (int64_t)colh * a.sdq_h + (int64_t)colt * a.sdq_t;
    typename Raw4<T>::type dq_prev[DK / 16];
    if (a.dq_acc) {
#pragma unroll
      for (int j = 0; j < DK / 16; ++j) dq_prev[j] = load4_raw<T>(dqp + j * 16 + 4 * g4);
    }
    const float sg = a.scale * rgate;
#pragma unroll
    for (int j = 0; j < DK / 16; ++j) {
      f32x4 v = dqa[j] * sg;
      if (a.dq_acc) v += raw4_f32(dq_prev[j]);
      store4<T>(dqp + j * 16 + 4 * g4, v);
    }
  }
}

template <typename T, int DK, int DV, int BR>
void launch_attn_bwd_dq(const AttnArgs& a, hipStream_t s) {
  if constexpr (BR == kSelection) {
    launch_attn_sel_dq<T, DK, DV>(a, s);  // per-wave selection kernel
  } else {
    using TL = DqTile<T, DK, DV>;
    const size_t lds = (size_t)TL::NBUF * TL::BYTES;
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_bwd_dq_kernel<T, DK, DV, BR>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    dim3 grid((a.Tq * a.hpg + kDqCols - 1) / kDqCols, a.B * a.G);
    hipLaunchKernelGGL((attn_bwd_dq_kernel<T, DK, DV, BR>), grid, dim3(64 * kDqWaves), lds, s, a);
  }
}

}  // namespace nsa
