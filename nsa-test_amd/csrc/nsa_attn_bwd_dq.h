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
// Workgroup = kDqWaves waves x kDqNSub x 16 query columns.  The operands of a 64-key tile --
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
// bf16 sliding window at head dims up to 64: capped at 80 registers (a 20-byte spill)
// so that two 12-wave workgroups share a CU (small launches fit in one round)
__global__ __launch_bounds__(64 * kDqWaves)
__attribute__((amdgpu_waves_per_eu(DK <= 64 && sizeof(T) == 2 && BR == kSliding ? 6 : 1)))
void attn_bwd_dq_kernel(AttnArgs a) {
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
  constexpr int NS = kDqNSub;  // 16-column subtiles per wave: each fragment read feeds NS products
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

  // NS 16-column subtiles per wave
  int colt[NS], colh[NS], sub_t0[NS], sub_t1[NS], kmin_s[NS];
  bool colv[NS], full[NS];
  uint32_t kspan_s[NS];
  int64_t srow[NS];
  uint4 qf[NS][NKC], dof[NS][NVC];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int f0 = col_base + (wave * NS + s) * 16;
    const int f = f0 + c16;
    colv[s] = f < ncols;
    full[s] = f0 + 16 <= ncols;
    colt[s] = colv[s] ? f / hpg : 0;
    colh[s] = colv[s] ? grp * hpg + f % hpg : 0;
    sub_t0[s] = f0 / hpg;
    sub_t1[s] = f0 < ncols ? min(a.Tq - 1, (f0 + 15) / hpg) : -1;
    const S* qp = reinterpret_cast<const S*>(a.q) + b * a.sq_b + (int64_t)colh[s] * a.sq_h + (int64_t)colt[s] * a.sq_t;
    const S* dp = reinterpret_cast<const S*>(a.dout) + b * a.sdo_b + (int64_t)colh[s] * a.sdo_h +
                  (int64_t)colt[s] * a.sdo_t;
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc)
      qf[s][kc] = colv[s] ? *reinterpret_cast<const uint4*>(qp + kc * KC + g4 * EPF) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int kc = 0; kc < NVC; ++kc)
      dof[s][kc] = colv[s] ? *reinterpret_cast<const uint4*>(dp + kc * KC + g4 * EPF) : make_uint4(0, 0, 0, 0);
    srow[s] = ((int64_t)b * a.H + colh[s]) * a.Tq + colt[s];
    // sliding: the column sees keys [kmin_s, kmin_s + kspan_s) (branch-free test)
    kmin_s[s] = max(colt[s] - a.window + 1, 0);
    kspan_s[s] = colv[s] ? (uint32_t)max(0, min(colt[s], a.Tkv - 1) + 1 - kmin_s[s]) : 0u;
  }

  f32x4 dqa[NS][DK / 16];
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int j = 0; j < DK / 16; ++j) dqa[s][j] = zero4();

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
      // issued past the compiler's wait insertion (which would make the tile's first LDS
      // read wait for this copy of the next tile); the loop waits for it before the
      // barrier that starts the next tile
      copy16_to_lds_async(src, dst + fr * 64);
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
  float l2[NS], dl[NS], rgate[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s)
    dq_row_stats<T, NVC>(a, b, colh[s], colt[s], colv[s], dof[s], g4, srow[s], l2[s], dl[s], rgate[s]);

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
    // between register files on every tile.  Each fragment read from LDS feeds the
    // products of all NS subtiles.
    f32x4 st[NS][4], dp[NS][4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        st[s][ks] = zero4();
        dp[s][ks] = zero4();
      }
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc) {
        const uint4 kf = kb[(ks * NKC + kc) * 64 + lane];
#pragma unroll
        for (int s = 0; s < NS; ++s) st[s][ks] = Mma<T>::run(st[s][ks], kf, qf[s][kc]);
      }
#pragma unroll
      for (int kc = 0; kc < NVC; ++kc) {
        const uint4 vf = vb[(ks * NVC + kc) * 64 + lane];
#pragma unroll
        for (int s = 0; s < NS; ++s) dp[s][ks] = Mma<T>::run(dp[s][ks], vf, dof[s][kc]);
      }
    }
    uint4 sf[NS][64 / CK];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      bool all_visible = false;
      if (BR == kSliding)
        all_visible = full[s] && key0 + 63 <= sub_t0[s] && key0 > sub_t1[s] - a.window && key0 + 63 < a.Tkv;
      else
        all_visible = full[s] && be_max <= sub_t0[s];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          bool ok = true;
          if (!all_visible) {
            const int key = key0 + ks * 16 + 4 * g4 + i;
            if (BR == kSliding) ok = (uint32_t)(key - kmin_s[s]) < kspan_s[s];
            else ok = colv[s] & (sbe[ks * 16 + 4 * g4 + i] <= colt[s]);
          }
          // the mask on the exponent argument: no divergent branch around the exp
          const float p = fast_exp2(ok ? st[s][ks][i] * scale2 - l2[s] : -INFINITY);
          st[s][ks][i] = p * (dp[s][ks][i] - dl[s]);  // dS^T
        }
      }
#pragma unroll
      for (int kc2 = 0; kc2 < 64 / CK; ++kc2) sf[s][kc2] = CFrag<T>::pack(st[s][kc2 * CT], st[s][kc2 * CT + CT - 1]);
    }
#pragma unroll
    for (int kc2 = 0; kc2 < 64 / CK; ++kc2) {
#pragma unroll
      for (int j = 0; j < DK / 16; ++j) {
        const uint4 tf = tb[(kc2 * (DK / 16) + j) * 64 + lane];
#pragma unroll
        for (int s = 0; s < NS; ++s) dqa[s][j] = Mma<T>::run(dqa[s][j], tf, sf[s][kc2]);
      }
    }
    if (TL::NBUF == 1 && it + 1 < ntiles) {  // single buffer: refill once every wave is done
      __syncthreads();
      copy_tile(tile_key0(it + 1), 0);
      load_be(tile_key0(it + 1));
    }
  }

#pragma unroll
  for (int s = 0; s < NS; ++s) {
    if (!colv[s]) continue;
    // accumulate mode: the caller's running dQ (loaded here, not at the start: the
    // registers are not spare in this kernel)
    S* dqp = reinterpret_cast<S*>(a.dq) + b * a.sdq_b + (int64_t)colh[s] * a.sdq_h + (int64_t)colt[s] * a.sdq_t;
    typename Raw4<T>::type dq_prev[DK / 16];
    if (a.dq_acc) {
#pragma unroll
      for (int j = 0; j < DK / 16; ++j) dq_prev[j] = load4_raw<T>(dqp + j * 16 + 4 * g4);
    }
    const float sg = a.scale * rgate[s];
#pragma unroll
    for (int j = 0; j < DK / 16; ++j) {
      f32x4 v = dqa[s][j] * sg;
      if (a.dq_acc) v += raw4_f32(dq_prev[j]);
      store4<T>(dqp + j * 16 + 4 * g4, v);
    }
  }
}

// ============================ dQ from the stored dS =============================
// Sliding window / compression, bf16, heads per group a multiple of 16, after the dK/dV
// kernel has stored dS per (timestep, 32-key chunk).  The workgroup walks the 64-key
// tiles of its columns' key span as the dQ kernel above does, with only the K^T
// colfrags of a tile in LDS (direct-to-LDS copies, double-buffered); each wave (the
// 16 heads of one head group at one timestep) reads its two stored dS fragments of the
// tile from HBM, one tile ahead, zeros for chunks its timestep does not see, and runs
// the one product dQ^T += K^T dS^T.  The stored dS carries the row gate: the epilogue
// scales by sm_scale only.  The sliding-window kernel can also run a compression
// branch's pass (pair_ds set: that backward's stored dS and K^T colfrags) into the same
// accumulators before its one epilogue, so the running dQ is read and written once for
// both branches.

// one branch's stored dS and K^T colfrags, as the dQ pass reads them
struct DqDsSource {
  const void* kcf;          // K^T colfrags, Tp rows per (batch, group)
  const void* ds;           // stored dS
  const int* block_ends;    // compression only
  int Tkv, Tp, ds_nch, window;
};

// One branch's tiles for the workgroup's columns, accumulated into dqa.  Every wave
// takes part (the copies are shared); wv: the wave owns columns.
template <typename T, int DK, int BR>
__device__ __forceinline__ void dq_ds_pass(const AttnArgs& a, const DqDsSource& src, uint4* lds, int* s_misc, int* s_cbe,
                                           int bg, int t, int hg, bool wv, int t_first, int t_last,
                                           f32x4 (&dqa)[DK / 16]) {
  using S = typename Store<T>::type;
  constexpr int EPF = Elem<T>::kPerFrag;
  constexpr int NW = kDqWaves;
  constexpr int NTF = 2 * (DK / 16);  // K^T colfrags of a 64-key tile (kc2, j)
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hpg = a.hpg;
  const S* kcf = reinterpret_cast<const S*>(src.kcf) + (int64_t)bg * DK * src.Tp;
  // the timestep's stored chunks: sliding [c_lo, c_hi]; compression those whose first
  // key is visible (block ends ascend)
  const int c_lo = BR == kSliding ? max(0, t - src.window + 1) >> 5 : 0;
  const int c_hi = BR == kSliding ? (min(t, src.Tkv - 1) >> 5) : 0x7fffffff;
  const S* dsb = reinterpret_cast<const S*>(src.ds) + (((int64_t)bg * a.Tq + t) * (hpg >> 4) + hg) * src.ds_nch * 512;

  int ntiles = 0, key_lo = 0;
  if (BR == kSliding) {
    key_lo = max(0, t_first - src.window + 1) & ~31;
    const int hi = min(t_last, src.Tkv - 1);
    ntiles = hi >= key_lo ? (hi - key_lo) / 64 + 1 : 0;
  } else {
    if (tid == 0) s_misc[0] = 0;
    __syncthreads();
    int mx = 0;
    for (int i = tid; i < src.Tkv; i += blockDim.x)
      if (src.block_ends[i] <= t_last) mx = i + 1;
    if (mx) atomicMax(&s_misc[0], mx);
    // the block end of each 32-key chunk's first key, read by the tile loop from LDS: a
    // global load there would make the wave wait for every load in flight before it
    for (int i = tid; i < (src.Tkv + 31) / 32; i += blockDim.x) s_cbe[i] = src.block_ends[i * 32];
    __syncthreads();
    ntiles = (s_misc[0] + 63) / 64;
  }
  auto tile_key0 = [&](int it) -> int { return BR == kSliding ? key_lo + it * 64 : it * 64; };
  auto copy_tile = [&](int key0, int buf) __attribute__((always_inline)) {
    uint4* dst = lds + buf * NTF * 64;
    for (int fr = wave; fr < NTF; fr += NW) {
      const int kc2 = fr / (DK / 16), j = fr % (DK / 16);
      // issued past the compiler's wait insertion, which would otherwise make the tile's
      // first LDS read wait for this copy and for the dS loads issued with it (the loop
      // waits for both itself, before the barrier that starts the next tile)
      copy16_to_lds_async(kcf + ((((int64_t)(key0 >> 5) + kc2) * (DK / 16) + j) * 64 + lane) * EPF,
                          dst + fr * 64);
    }
  };
  // the wave's dS fragments of the tile at key0 (zero for chunks it does not see)
  auto load_ds = [&](int key0, u32x4 (&df)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int kc2 = 0; kc2 < 2; ++kc2) {
      const int kg = (key0 >> 5) + kc2;
      bool vis = wv && kg >= c_lo && kg <= c_hi && kg * 32 < src.Tkv;
      if (BR == kCompression && vis) vis = s_cbe[kg] <= t;
      df[kc2] = vis ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(dsb + (int64_t)(kg - c_lo) * 512 + lane * EPF))
                    : u32x4{0u, 0u, 0u, 0u};
    }
  };

  u32x4 df[2], dfn[2];
  if (ntiles > 0) {
    copy_tile(tile_key0(0), 0);
    load_ds(tile_key0(0), df);
  }
  for (int it = 0; it < ntiles; ++it) {
    const int buf = it & 1;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's copies of tile it (and its dS) have landed
    __syncthreads();                // every wave's have; tile it-1 is no longer read
    if (it + 1 < ntiles) {
      copy_tile(tile_key0(it + 1), buf ^ 1);
      load_ds(tile_key0(it + 1), dfn);
    }
    const uint4* tb = lds + buf * NTF * 64;
#pragma unroll
    for (int kc2 = 0; kc2 < 2; ++kc2)
#pragma unroll
      for (int j = 0; j < DK / 16; ++j)
        dqa[j] = Mma<T>::run(dqa[j], tb[(kc2 * (DK / 16) + j) * 64 + lane], __builtin_bit_cast(uint4, df[kc2]));
    df[0] = dfn[0];
    df[1] = dfn[1];
  }
}

template <typename T, int DK, int BR>
__global__ __launch_bounds__(64 * kDqWaves) void attn_bwd_dq_ds_kernel(AttnArgs a) {
  static_assert(BR == kSliding || BR == kCompression, "dense branches");
  using S = typename Store<T>::type;
  static_assert(sizeof(S) == 2, "stored dS is bf16");
  extern __shared__ __attribute__((aligned(16))) uint4 dqds_lds[];  // [2][2 DK / 16][64]
  __shared__ int s_misc[4];
  __shared__ int s_cbe[kDqCbeMax];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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

  // the wave's 16 columns: one head group at one timestep
  const int f0 = col_base + wave * 16;
  const bool wv = f0 < ncols;
  const int t = wv ? f0 / hpg : t_first;
  const int hg = (f0 - t * hpg) >> 4;
  const int colh = grp * hpg + (f0 - t * hpg) + c16;

  f32x4 dqa[DK / 16];
#pragma unroll
  for (int j = 0; j < DK / 16; ++j) dqa[j] = zero4();
  const DqDsSource own{a.kcf, a.ds, a.block_ends, a.Tkv, a.Tp, a.ds_nch, a.window};
  dq_ds_pass<T, DK, BR>(a, own, dqds_lds, s_misc, s_cbe, bg, t, hg, wv, t_first, t_last, dqa);
  if constexpr (BR == kSliding) {
    if (a.pair_ds) {
      __syncthreads();  // every wave is past the last tile of the first pass
      const DqDsSource pair{a.pair_kcf, a.pair_ds, a.pair_block_ends, a.pair_Tkv, a.pair_Tp, a.pair_ds_nch, 0};
      dq_ds_pass<T, DK, kCompression>(a, pair, dqds_lds, s_misc, s_cbe, bg, t, hg, wv, t_first, t_last, dqa);
    }
  }
  if (!wv) return;
  S* dqp = reinterpret_cast<S*>(a.dq) + b * a.sdq_b + (int64_t)colh * a.sdq_h + (int64_t)t * a.sdq_t;
#pragma unroll
  for (int j = 0; j < DK / 16; ++j) {
    f32x4 v = dqa[j] * a.scale;
    if (a.dq_acc) v += load4<T>(dqp + j * 16 + 4 * g4);  // the caller's running dQ sum
    store4<T>(dqp + j * 16 + 4 * g4, v);
  }
}

template <typename T, int DK, int DV, int BR>
void launch_attn_bwd_dq(const AttnArgs& a, hipStream_t s) {
  if constexpr (BR == kSelection) {
    launch_attn_sel_dq<T, DK, DV>(a, s);  // per-wave selection kernel
  } else {
    if constexpr (sizeof(typename Store<T>::type) == 2) {
      if (a.ds) {
        const size_t lds = (size_t)2 * 2 * (DK / 16) * 1024;
        allow_dynamic_lds(reinterpret_cast<const void*>(&attn_bwd_dq_ds_kernel<T, DK, BR>), lds);
        dim3 grid((a.Tq * a.hpg + kDqCols - 1) / kDqCols, a.B * a.G);
        hipLaunchKernelGGL((attn_bwd_dq_ds_kernel<T, DK, BR>), grid, dim3(64 * kDqWaves), lds, s, a);
        return;
      }
    }
    using TL = DqTile<T, DK, DV>;
    const size_t lds = (size_t)TL::NBUF * TL::BYTES;
    allow_dynamic_lds(reinterpret_cast<const void*>(&attn_bwd_dq_kernel<T, DK, DV, BR>), lds);
    dim3 grid((a.Tq * a.hpg + kDqCols - 1) / kDqCols, a.B * a.G);
    hipLaunchKernelGGL((attn_bwd_dq_kernel<T, DK, DV, BR>), grid, dim3(64 * kDqWaves), lds, s, a);
  }
}

}  // namespace nsa
