// Top-n block selection attention, forward and dQ, on gfx950.
//
// Each wave is independent: it owns 16 query columns ((timestep, head) pairs of one
// KV group; with 16 heads per group, one timestep) and walks the union of the blocks
// its timesteps selected.  K and V fragments are read straight from the re-packed
// group K/V (kt [T][dk], kn [dk][T], vt [dv][T], vn [T][dv]) into MFMA operand
// registers -- no LDS staging and no workgroup barrier -- so a wave never waits for
// blocks another wave's timesteps chose, and blocks shared by neighbouring timesteps
// (the fixed initial / local blocks, correlated top-n) are served by L2.  Workgroups
// are mapped XCD-contiguously so that neighbouring timesteps share an L2.
//
// Key j is visible to column (t, h) iff j lies in a block the row selected (the
// cleaned, de-duplicated list), j < N_CTX_KV and (causal) j <= t
// (reference nsa/reference.py:205-254).
#pragma once
#include "nsa_attn.h"
#include "nsa_device.h"
#include "nsa_attn_rowstats.h"

namespace nsa {

constexpr int kSelWaveCols = 16;
constexpr int kSelMaxT = 17;  // timesteps a 16-column group can touch (hpg = 1)

// Workgroup id -> logical id such that each XCD (ids dispatched round-robin over 8)
// receives a contiguous range of logical ids.
__device__ __forceinline__ int xcd_contiguous(int i, int n) {
  const int xcd = i & 7, k = i >> 3;
  const int base = n >> 3, rem = n & 7;
  return (xcd < rem ? xcd * (base + 1) : rem * (base + 1) + (xcd - rem) * base) + k;
}

// Per-wave bookkeeping: the timesteps of the wave's columns, their cleaned lists and
// the union bitmap of their blocks.
struct SelWave {
  int t_first, nt;
};

template <typename T, bool DQ>
__device__ __forceinline__ void sel_wave_setup(const AttnArgs& a, int bg, int f0, int* lst, uint32_t* bits,
                                               SelWave& w, int lane) {
  const int ncols = a.Tq * a.hpg;
  const int flast = min(f0 + kSelWaveCols, ncols) - 1;
  w.t_first = f0 / a.hpg;
  w.nt = flast / a.hpg - w.t_first + 1;
  const int nwords = (a.nblk + 31) / 32;
  for (int i = lane; i < nwords; i += 64) bits[i] = 0;
  __builtin_amdgcn_wave_barrier();
  const int* selrow = a.sel + ((int64_t)bg * a.Tq + w.t_first) * a.nslots;
  const int total = w.nt * a.nslots;
  for (int i = lane; i < total; i += 64) {
    const int v = selrow[i];
    lst[i] = v;
    if (v >= 0) atomicOr(&bits[v >> 5], 1u << (v & 31));
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
}

// does the column's timestep select block `blk`? (its list is ascending, -1 padded)
__device__ __forceinline__ bool sel_has(const int* l, int nslots, int blk) {
  bool has = false;
  for (int j = 0; j < nslots; ++j) {
    const int v = l[j];
    if (v == blk) has = true;
    if (v < 0 || v >= blk) break;
  }
  return has;
}

// ============================================================== forward
// Two phases.  (1) bf16: the blocks every wave of the workgroup selected (at 16 heads per
// group: the four timesteps' common blocks -- block 0 and the local ones at least) are
// walked by the whole workgroup: each tile's K / V^T fragments are copied direct-to-LDS
// once and all four waves compute from them.  (2) Every wave walks the rest of its
// union on its own, fragments straight from L2 into registers one tile ahead.  Both
// phases feed the same online softmax; every column applies its own selection mask in
// both.
template <typename T, int DK, int DV>
struct SelFwdShared {
  static constexpr int KC = Elem<T>::kKChunk;
  static constexpr int CK = CFrag<T>::kKeys;
  static constexpr int NKF = 4 * (DK / KC);          // K rowfrags of a 64-key tile
  static constexpr int NVF = (64 / CK) * (DV / 16);  // V^T colfrags
  static constexpr bool kOn = sizeof(typename Store<T>::type) == 2;
  static constexpr int kLdsBytes = kOn ? (NKF + NVF) * 1024 : 0;
};

template <typename T, int DK, int DV>
// Two waves per SIMD (256 registers): the second wave covers the latency of the first
// one's fragment loads and softmax, which bound this kernel with one wave per SIMD.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void attn_sel_fwd_kernel(AttnArgs a, int ncoltiles) {
  using S = typename Store<T>::type;
  using SH = SelFwdShared<T, DK, DV>;
  constexpr int EPF = Elem<T>::kPerFrag;
  constexpr int KC = Elem<T>::kKChunk;
  constexpr int NKC = DK / KC;
  constexpr int CK = CFrag<T>::kKeys;
  constexpr int CT = CK / 16;
  constexpr int NWD = kSelMaxBlocks / 32;
  __shared__ int s_lst[4][kSelMaxT * 64];
  __shared__ uint32_t s_bits[4][NWD];
  extern __shared__ __attribute__((aligned(16))) uint4 sel_tile[];  // [NKF + NVF][64] (phase 1)

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform control below
  const int g4 = lane >> 4, c16 = lane & 15;
  const int L = xcd_contiguous(blockIdx.x, gridDim.x);
  const int bg = L / ncoltiles;
  const int b = bg / a.G, grp = bg % a.G;
  const int hpg = a.hpg;
  const int ncols = a.Tq * hpg;
  const int f0 = (L % ncoltiles) * 64 + wave * kSelWaveCols;
  const bool active = f0 < ncols;  // idle waves still meet the phase-1 barriers
  const float scale2 = a.scale * kLog2e;
  const int nwords = (a.nblk + 31) / 32;

  SelWave w{0, 0};
  int* lst = s_lst[wave];
  uint32_t* bits = s_bits[wave];
  if (active) {
    sel_wave_setup<T, false>(a, bg, f0, lst, bits, w, lane);
  } else if (SH::kOn) {
    for (int i = lane; i < nwords; i += 64) bits[i] = 0;
  }

  const int f = f0 + c16;
  const bool colv = active && f < ncols;
  const int colt = colv ? f / hpg : w.t_first;
  const int colh = colv ? grp * hpg + f % hpg : grp * hpg;
  const int t_last = w.t_first + w.nt - 1 + a.q0;  // absolute positions: row r is at a.q0 + r
  const int* mylst = lst + (colt - w.t_first) * a.nslots;

  const S* qp = reinterpret_cast<const S*>(a.q) + b * a.sq_b + (int64_t)colh * a.sq_h + (int64_t)colt * a.sq_t;
  uint4 qf[NKC];
#pragma unroll
  for (int kc = 0; kc < NKC; ++kc)
    qf[kc] = colv ? *reinterpret_cast<const uint4*>(qp + kc * KC + g4 * EPF) : make_uint4(0, 0, 0, 0);

  const S* krf = reinterpret_cast<const S*>(a.krf) + (int64_t)bg * a.Tp * DK;
  const S* vcf = reinterpret_cast<const S*>(a.vcf) + (int64_t)bg * DV * a.Tp;
  f32x4 oacc[DV / 16];
#pragma unroll
  for (int j = 0; j < DV / 16; ++j) oacc[j] = zero4();
  float m2 = -INFINITY, mtrue = -INFINITY, lsum = 0.f;  // exponent reference, true maximum, sum
  const bool one_t = w.nt == 1;

  // masking and the online softmax of one tile's S^T (keys key0 .. key0 + 63 of block blk
  // [blk_lo, blk_hi)); returns the packed P^T fragments
  auto softmax_tile = [&](f32x4 (&st)[4], int key0, int blk, int blk_hi, uint4 (&pf)[64 / CK])
                          __attribute__((always_inline)) {
    const int blk_lo = blk * a.lprime;
    const bool colsel = colv && (one_t || sel_has(mylst, a.nslots, blk));
    // end of the keys of this block the lane's column sees (blk_lo when none)
    const int kend = colsel ? max(blk_lo, a.causal ? min(blk_hi, colt + a.q0 + 1) : blk_hi) : blk_lo;
    const bool all_visible = one_t && colv && (!a.causal || key0 + 63 <= w.t_first + a.q0) && key0 >= blk_lo &&
                             key0 + 63 < blk_hi && f0 + kSelWaveCols <= ncols;
    float mx = -INFINITY;
    // lane-visible keys of this block: [blk_lo, kend); branch-free test per element
    const uint32_t span = all_visible ? 0xffffffffu : (uint32_t)(kend - blk_lo);
    const int kb = key0 + 4 * g4 - blk_lo;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool ok = (uint32_t)(kb + ks * 16 + i) < span;
        const float v = ok ? st[ks][i] : -INFINITY;
        st[ks][i] = v;
        mx = fmaxf(mx, v);
      }
    // maximum over the raw products (scale2 > 0; the exponent argument is the rounded
    // product minus the reference, so the maximum maps to exp2(0) = 1 exactly); lazy
    // rescale of the exponent reference m2 (moves only when a column maximum exceeds it
    // by kLazyRescale), the true maximum mtrue kept for M and the epilogue
    mx = wave_max16(mx) * scale2;
    mtrue = fmaxf(mtrue, mx);
    if (__ballot(mx > m2 + kLazyRescale) != 0ull) {
      const float mnew = fmaxf(m2, mtrue);
      const float alpha = m2 == -INFINITY ? 0.f : fast_exp2(m2 - mnew);
      lsum *= alpha;
#pragma unroll
      for (int j = 0; j < DV / 16; ++j) oacc[j] *= alpha;
      m2 = mnew;
    }
    const float nref = m2 == -INFINITY ? 0.f : -m2;
    float rs = 0.f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = fast_exp2(mul_add_rounded(st[ks][i], scale2, nref));
        st[ks][i] = p;
        rs += p;
      }
    lsum += wave_sum16(rs);
#pragma unroll
    for (int kc2 = 0; kc2 < 64 / CK; ++kc2) pf[kc2] = CFrag<T>::pack(st[kc2 * CT], st[kc2 * CT + CT - 1]);
  };

  // ---- phase 1: the workgroup's common blocks, one LDS copy per tile -----------------
  __shared__ uint32_t s_common[SH::kOn ? NWD : 1];
  if constexpr (SH::kOn) {
    __syncthreads();  // every wave's bitmap is written
    for (int i = threadIdx.x; i < nwords; i += 256) s_common[i] = s_bits[0][i] & s_bits[1][i] & s_bits[2][i] & s_bits[3][i];
    __syncthreads();
    const int t_max = (min((L % ncoltiles) * 64 + 64, ncols) - 1) / hpg + a.q0;  // the workgroup's last position
    for (int wd = 0; wd < nwords; ++wd) {
      uint32_t word = s_common[wd];  // uniform across the workgroup
      while (word) {
        const int blk = wd * 32 + __builtin_ctz(word);
        word &= word - 1;
        const int lo = blk * a.lprime;
        const int blk_hi = min(lo + a.lprime, a.Tkv);
        for (int key0 = lo & ~31; key0 < blk_hi && !(a.causal && key0 > t_max); key0 += 64) {
          for (int fr = wave; fr < SH::NKF + SH::NVF; fr += 4) {
            const S* src;
            if (fr < SH::NKF) {
              const int ks = fr / NKC, kc = fr % NKC;
              src = krf + ((((int64_t)(key0 >> 4) + ks) * NKC + kc) * 64 + lane) * EPF;
            } else {
              const int v = fr - SH::NKF, kc2 = v / (DV / 16), j = v % (DV / 16);
              src = vcf + ((((int64_t)(key0 / CK) + kc2) * (DV / 16) + j) * 64 + lane) * EPF;
            }
            copy16_to_lds(src, sel_tile + fr * 64);
          }
          __builtin_amdgcn_s_waitcnt(0);
          __syncthreads();
          if (active) {
            f32x4 st[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
              st[ks] = zero4();
#pragma unroll
              for (int kc = 0; kc < NKC; ++kc) st[ks] = Mma<T>::run(st[ks], sel_tile[(ks * NKC + kc) * 64 + lane], qf[kc]);
            }
            uint4 pf[64 / CK];
            softmax_tile(st, key0, blk, blk_hi, pf);
#pragma unroll
            for (int kc2 = 0; kc2 < 64 / CK; ++kc2)
#pragma unroll
              for (int j = 0; j < DV / 16; ++j)
                oacc[j] = Mma<T>::run(oacc[j], sel_tile[(SH::NKF + kc2 * (DV / 16) + j) * 64 + lane], pf[kc2]);
          }
          __syncthreads();  // the tile is read before the next copy
        }
      }
    }
  }
  if (!active) return;

  // ---- phase 2: the rest of the wave's union, straight from L2 --------------------------
  // Tile cursor over the union bitmap (wave-uniform scalar state).  Tiles start on a
  // 32-key boundary (the C-permuted chunks of vt / kn) and cover 64 keys.
  int c_wd = -1, c_blk = -1, c_key0 = 0, c_hi = 0;
  uint32_t c_word = 0;
  auto advance = [&]() -> bool {
    if (c_blk >= 0) {
      c_key0 += 64;
      if (c_key0 < c_hi && !(a.causal && c_key0 > t_last)) return true;
    }
    while (c_word == 0) {
      if (++c_wd >= nwords) return false;
      uint32_t wd = bits[c_wd];
      if constexpr (SH::kOn) wd &= ~s_common[c_wd];
      c_word = __builtin_amdgcn_readfirstlane(wd);
    }
    c_blk = c_wd * 32 + __builtin_ctz(c_word);
    c_word &= c_word - 1;
    const int lo = c_blk * a.lprime;
    c_hi = min(lo + a.lprime, a.Tkv);
    c_key0 = lo & ~31;
    return true;
  };
  // K fragments of a tile (S^T = K Q^T) and V^T fragments (O^T += V^T P^T): the next
  // tile's K is requested as soon as the current S^T is issued, its V as soon as the
  // current P V is, so the loads overlap the softmax and the products.
  uint4 kf[4][NKC], vf[64 / CK][DV / 16];
  auto load_k = [&](int key0) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc)
        kf[ks][kc] = ld_rowfrag<T>(krf, (key0 >> 4) + ks, kc, DK, lane);
  };
  auto load_v = [&](int key0) {
#pragma unroll
    for (int kc2 = 0; kc2 < 64 / CK; ++kc2)
#pragma unroll
      for (int j = 0; j < DV / 16; ++j)
        vf[kc2][j] = ld_colfrag<T>(vcf, key0 / CK + kc2, j, DV, lane);
  };

  bool have = advance();
  if (have) {
    load_k(c_key0);
    load_v(c_key0);
  }
  while (have) {
    const int key0 = c_key0, blk = c_blk;
    const int blk_hi = c_hi;
    // S^T[key, col] for the 64 keys of this tile
    f32x4 st[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      st[ks] = zero4();
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc) st[ks] = Mma<T>::run(st[ks], kf[ks][kc], qf[kc]);
    }
    const bool have_next = advance();
    if (have_next) load_k(c_key0);
    uint4 pf[64 / CK];
    softmax_tile(st, key0, blk, blk_hi, pf);
#pragma unroll
    for (int kc2 = 0; kc2 < 64 / CK; ++kc2) {
#pragma unroll
      for (int j = 0; j < DV / 16; ++j) oacc[j] = Mma<T>::run(oacc[j], vf[kc2][j], pf[kc2]);
    }
    if (have_next) load_v(c_key0);
    have = have_next;
  }

  if (colv) {
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    if (lsum > 0.f) lsum *= fast_exp2(m2 - mtrue);  // the sum relative to the true maximum
    S* op = reinterpret_cast<S*>(a.o) + b * a.so_b + (int64_t)colh * a.so_h + (int64_t)colt * a.so_t;
#pragma unroll
    for (int j = 0; j < DV / 16; ++j) store4<T>(op + j * 16 + 4 * g4, oacc[j] * inv);
    if (g4 == 0) {
      if (a.L)
        a.L[b * a.sl_b + (int64_t)colh * a.sl_h + (int64_t)colt * a.sl_t] = lsum > 0.f ? logf(lsum) : -INFINITY;
      if (a.M) a.M[b * a.sm_b + (int64_t)colh * a.sm_h + (int64_t)colt * a.sm_t] = mtrue * kLn2;
    }
  }
}

template <typename T, int DK, int DV>
void launch_attn_sel_fwd(const AttnArgs& a, hipStream_t s) {
  using SH = SelFwdShared<T, DK, DV>;
  const int ncoltiles = (a.Tq * a.hpg + 63) / 64;
  if (SH::kLdsBytes > 0)
    allow_dynamic_lds(reinterpret_cast<const void*>(&attn_sel_fwd_kernel<T, DK, DV>), SH::kLdsBytes);
  hipLaunchKernelGGL((attn_sel_fwd_kernel<T, DK, DV>), dim3(ncoltiles * a.B * a.G), dim3(256), SH::kLdsBytes, s, a,
                     ncoltiles);
}

// ============================================================== dQ
template <typename T, int DK, int DV>
__global__ __launch_bounds__(256) void attn_sel_dq_kernel(AttnArgs a, int ncoltiles) {
  using S = typename Store<T>::type;
  constexpr int EPF = Elem<T>::kPerFrag;
  constexpr int KC = Elem<T>::kKChunk;
  constexpr int NKC = DK / KC;
  constexpr int NVC = DV / KC;
  constexpr int CK = CFrag<T>::kKeys;
  constexpr int CT = CK / 16;
  __shared__ int s_lst[4][kSelMaxT * 64];
  __shared__ uint32_t s_bits[4][kSelMaxBlocks / 32];
  // bf16: each wave's staged K rows of one 64-key tile (rowfrag order)
  __shared__ __attribute__((aligned(16))) uint4 s_kt[4][sizeof(S) == 2 ? 4 * NKC * 64 : 1];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform control below
  const int g4 = lane >> 4, c16 = lane & 15;
  const int L = xcd_contiguous(blockIdx.x, gridDim.x);
  const int bg = L / ncoltiles;
  const int b = bg / a.G, grp = bg % a.G;
  const int hpg = a.hpg;
  const int ncols = a.Tq * hpg;
  const int f0 = (L % ncoltiles) * 64 + wave * kSelWaveCols;
  if (f0 >= ncols) return;
  const float scale2 = a.scale * kLog2e;

  SelWave w;
  int* lst = s_lst[wave];
  uint32_t* bits = s_bits[wave];
  sel_wave_setup<T, true>(a, bg, f0, lst, bits, w, lane);

  const int f = f0 + c16;
  const bool colv = f < ncols;
  const int colt = colv ? f / hpg : w.t_first;
  const int colh = colv ? grp * hpg + f % hpg : grp * hpg;
  const int t_last = w.t_first + w.nt - 1;
  const int* mylst = lst + (colt - w.t_first) * a.nslots;

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
  // accumulate mode: the caller's running dQ of the column, requested now (bf16; fp32 has
  // no spare registers and loads it in the epilogue) so that the load is complete by the
  // epilogue: with one wave per SIMD nothing else would hide its latency
  constexpr bool kPrefetchDq = sizeof(S) == 2;
  typename Raw4<T>::type dq_prev[DK / 16];
  S* dqp = reinterpret_cast<S*>(a.dq) + b * a.sdq_b + (int64_t)colh * a.sdq_h + (int64_t)colt * a.sdq_t;
  if (kPrefetchDq && a.dq_acc && colv) {
#pragma unroll
    for (int j = 0; j < DK / 16; ++j) dq_prev[j] = load4_raw<T>(dqp + j * 16 + 4 * g4);
  }

  const S* krf = reinterpret_cast<const S*>(a.krf) + (int64_t)bg * a.Tp * DK;
  const S* kcf = reinterpret_cast<const S*>(a.kcf) + (int64_t)bg * DK * a.Tp;
  const S* vrf = reinterpret_cast<const S*>(a.vrf) + (int64_t)bg * a.Tp * DV;
  f32x4 dqa[DK / 16];
#pragma unroll
  for (int j = 0; j < DK / 16; ++j) dqa[j] = zero4();
  const int nwords = (a.nblk + 31) / 32;
  const bool one_t = w.nt == 1;

  // wave-uniform tile cursor over the union bitmap (as in the forward)
  int c_wd = -1, c_blk = -1, c_key0 = 0, c_hi = 0;
  uint32_t c_word = 0;
  auto advance = [&]() -> bool {
    if (c_blk >= 0) {
      c_key0 += 64;
      if (c_key0 < c_hi && !(a.causal && c_key0 > t_last)) return true;
    }
    while (c_word == 0) {
      if (++c_wd >= nwords) return false;
      c_word = __builtin_amdgcn_readfirstlane(bits[c_wd]);
    }
    c_blk = c_wd * 32 + __builtin_ctz(c_word);
    c_word &= c_word - 1;
    const int lo = c_blk * a.lprime;
    c_hi = min(lo + a.lprime, a.Tkv);
    c_key0 = lo & ~31;
    return true;
  };
  // K and V rowfrags of a tile feed S^T = K Q^T and dP^T = V dO^T; K^T fragments feed
  // dQ^T += K^T dS^T.
  //  bf16: the K rows of a tile go to the wave's own LDS region by direct-to-LDS loads
  //    (24 KB at dk = 192); the rowfrags are read back as they are and the K^T fragments
  //    with the LDS transpose load, so each (timestep, block) pair gathers K once (40
  //    instead of 64 KB from L2 with V).  All of them are read into registers when the
  //    tile starts, which frees the region for the next tile's copy at once.
  //  fp32: K colfrags are read from the re-packed K^T (kcf) once S^T / dP^T are issued.
  // The next tile's loads are issued once this tile's S^T and dP^T are, so they overlap
  // the softmax and the dQ products.
  constexpr bool kLdsK = sizeof(S) == 2;
  constexpr int NVL = 4 * NVC;  // V fragment loads per tile
  uint4 kf[4][NKC], vf[4][NVC], knf[64 / CK][DK / 16];
  uint4* kst = s_kt[wave];
  auto load_k = [&](int key0) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc) {
        if constexpr (kLdsK)
          copy16_to_lds(krf + ((((int64_t)(key0 >> 4) + ks) * NKC + kc) * 64 + lane) * EPF, kst + (ks * NKC + kc) * 64);
        else
          kf[ks][kc] = ld_rowfrag<T>(krf, (key0 >> 4) + ks, kc, DK, lane);
      }
  };
  auto load_v = [&](int key0) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int kc = 0; kc < NVC; ++kc) vf[ks][kc] = ld_rowfrag<T>(vrf, (key0 >> 4) + ks, kc, DV, lane);
  };
  // K^T fragment (32-key chunk kc2, features 16j..16j+15) from the staged rowfrags:
  // lane (g4, f) needs K[key][16j + f] for keys 4g4..4g4+3 and 16+4g4..16+4g4+3 of the
  // chunk (the C-permuted order); the transpose load gives each 16-lane group a 4-key x
  // 16-feature block whose row rho is key 4g4+rho, lanes 4rho+q reading its features
  // 4q..4q+3: in rowfrag (16-key group ks, chunk kc) feature e of key r sits at lane
  // ((e % 32) / 8) * 16 + r, element e % 8.
  auto knf_lds = [&](int kc2, int j) -> uint4 {
    const int rho = c16 >> 2, q = c16 & 3;
    const int e = 16 * j + 4 * q;  // first of the lane's four features
    const int kc = e / KC, gp = (e % KC) / EPF, el = e % EPF;
    const uint16_t* base = reinterpret_cast<const uint16_t*>(kst);
    const int r = 4 * g4 + rho;
    const uint16_t* p0 = base + (((2 * kc2) * NKC + kc) * 64 + gp * 16 + r) * EPF + el;
    return ld_tr_pair(p0, NKC * 64 * EPF);  // second half: the next 16-key group
  };
  // bf16: the tile's K copy (issued before its V loads) has landed once at most NVL
  // vector-memory operations are outstanding; read every K and K^T fragment of the tile
  // into registers, then the region is free for the next tile's copy.
  auto fetch_k = [&]() {
    if constexpr (kLdsK) {
      wait_vmcnt<NVL>();
      __builtin_amdgcn_wave_barrier();
      asm volatile("" ::: "memory");
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int kc = 0; kc < NKC; ++kc) kf[ks][kc] = kst[(ks * NKC + kc) * 64 + lane];
#pragma unroll
      for (int kc2 = 0; kc2 < 64 / CK; ++kc2)
#pragma unroll
        for (int j = 0; j < DK / 16; ++j) knf[kc2][j] = knf_lds(kc2, j);
      wave_lds_sync();
      asm volatile("" ::: "memory");
    }
  };
  bool have = advance();
  if (have) {
    load_k(c_key0);
    load_v(c_key0);
  }
  // row statistics after the first tile's loads are issued (their O loads overlap them)
  float l2, dl, rgate;
  dq_row_stats<T, NVC>(a, b, colh, colt, colv, dof, g4, srow, l2, dl, rgate);
  while (have) {
    const int key0 = c_key0, blk = c_blk;
    const int blk_lo = blk * a.lprime;
    const int blk_hi = c_hi;
    fetch_k();
    const bool have_next = advance();
    // the next tile's loads are unconditional (the last tile re-reads its own keys):
    // a branch around them would make the compiler wait for every outstanding load at
    // the join.  bf16: the K copy goes out now, a whole tile ahead of its use.
    const int next_key0 = have_next ? c_key0 : key0;
    if (kLdsK) load_k(next_key0);
    f32x4 st[4], dp[4];
    // S^T first (its operands are in registers), then dP^T, whose V rows may still be
    // arriving
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      st[ks] = zero4();
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc) st[ks] = Mma<T>::run(st[ks], kf[ks][kc], qf[kc]);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      dp[ks] = zero4();
#pragma unroll
      for (int kc = 0; kc < NVC; ++kc) dp[ks] = Mma<T>::run(dp[ks], vf[ks][kc], dof[kc]);
    }
    if constexpr (!kLdsK) {
#pragma unroll
      for (int kc2 = 0; kc2 < 64 / CK; ++kc2)
#pragma unroll
        for (int j = 0; j < DK / 16; ++j) knf[kc2][j] = ld_colfrag<T>(kcf, key0 / CK + kc2, j, DK, lane);
      load_k(next_key0);
    }
    load_v(next_key0);

    const bool colsel = colv && (one_t || sel_has(mylst, a.nslots, blk));
    // end of the keys of this block the lane's column sees (blk_lo when none)
    const int kend = colsel ? max(blk_lo, a.causal ? min(blk_hi, colt + 1) : blk_hi) : blk_lo;
    const bool all_visible = one_t && colv && (!a.causal || key0 + 63 <= w.t_first) && key0 >= blk_lo &&
                             key0 + 63 < blk_hi && f0 + kSelWaveCols <= ncols;
    const uint32_t span = all_visible ? 0xffffffffu : (uint32_t)(kend - blk_lo);
    const int kb = key0 + 4 * g4 - blk_lo;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool ok = (uint32_t)(kb + ks * 16 + i) < span;
        const float p = fast_exp2(ok ? st[ks][i] * scale2 - l2 : -INFINITY);
        st[ks][i] = p * (dp[ks][i] - dl);  // dS^T
      }
#pragma unroll
    for (int kc2 = 0; kc2 < 64 / CK; ++kc2) {
      const uint4 sf = CFrag<T>::pack(st[kc2 * CT], st[kc2 * CT + CT - 1]);
#pragma unroll
      for (int j = 0; j < DK / 16; ++j) dqa[j] = Mma<T>::run(dqa[j], knf[kc2][j], sf);
    }
    have = have_next;
  }

  if (colv) {
    if (!kPrefetchDq && a.dq_acc) {
#pragma unroll
      for (int j = 0; j < DK / 16; ++j) dq_prev[j] = load4_raw<T>(dqp + j * 16 + 4 * g4);
    }
    const float sg = a.scale * rgate;
#pragma unroll
    for (int j = 0; j < DK / 16; ++j) {
      f32x4 v = dqa[j] * sg;
      if (a.dq_acc) v += raw4_f32(dq_prev[j]);  // the caller's running dQ sum
      store4<T>(dqp + j * 16 + 4 * g4, v);
    }
  }
}

// ============================================================== dQ from stored dS
// bf16, heads per group a multiple of 16, l' a multiple of 64, after the dK/dV kernel
// has stored every (timestep, slot) pair's dS (nsa_attn_bwd_dkdv.h): one wave = the 16
// heads of one head group at one timestep, dQ^T += K^T dS^T over the 64-key sub-blocks
// of the timestep's cleaned list (ascending; the visible ones form a prefix of the
// (slot, sub-block) order).  Both operands are fragment-native in memory -- K^T from
// the re-packed colfrag copy, dS^T as stored -- so every fragment is one coalesced 1 KB
// load: no S / dP recomputation, no softmax.  The K^T fragments go straight into
// registers; the next tile's fragments of one 32-key chunk are requested as soon as
// this tile's products have read that chunk.
//
// A wave's vector-memory loads complete in issue order, so a dS load from HBM placed
// between the K^T loads (L2 hits) would make every K^T load behind it wait for the HBM
// round trip.  The dS fragments of kDsBatch tiles are therefore copied direct-to-LDS
// in one batch, a batch ahead (two buffers per wave): one HBM round trip per batch
// instead of one per chunk.  The buffer after the last batch receives the dQ rows the
// result is added to (accumulate mode), so their HBM round trip overlaps the last
// batch's tiles instead of following them.  The stored dS already carries the row
// gate, so the epilogue scales by sm_scale only.
constexpr int kDsBatch = 3;
template <typename T, int DK>
__global__ __launch_bounds__(256) void attn_sel_dq_ds_kernel(AttnArgs a, int nwaves, int acc_lds) {
  using S = typename Store<T>::type;
  constexpr int EPF = Elem<T>::kPerFrag;
  static_assert(sizeof(S) == 2, "stored dS is bf16");
  static_assert(DK * 16 * 2 <= kDsBatch * 2 * 1024, "a buffer holds the wave's dQ rows");
  // per wave: two buffers of kDsBatch tiles x 2 chunks x 64 lanes x 16 bytes
  __shared__ uint4 s_ds[4][2][kDsBatch * 2][64];
  const int lane = threadIdx.x & 63;
  const int g4 = lane >> 4, c16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = xcd_contiguous(blockIdx.x, gridDim.x) * 4 + wave;
  if (W >= nwaves) return;
  const int nhg = a.hpg >> 4, nsub = a.lprime >> 6;
  const int per_bg = a.Tq * nhg;
  const int bg = W / per_bg, rem = W - bg * per_bg;
  const int t = rem / nhg, hg = rem - t * nhg;
  const int b = bg / a.G, grp = bg % a.G;
  const int colh = grp * a.hpg + hg * 16 + c16;

  // the timestep's cleaned list (lane s holds slot s) and its visible tile count: slot s
  // contributes the sub-blocks of its block that start before kend
  const int lv = lane < a.nslots ? a.sel[((int64_t)bg * a.Tq + t) * a.nslots + lane] : -1;
  const int kend = a.causal ? min(a.Tkv, t + 1) : a.Tkv;
  int nt = 0;
  if (lv >= 0) nt = min(nsub, max(0, (kend - lv * a.lprime + 63) >> 6));
  nt = __builtin_amdgcn_readfirstlane(wave_butterfly(nt, [](int x, int y) { return x + y; }));

  const S* kcf = reinterpret_cast<const S*>(a.kcf) + (int64_t)bg * DK * a.Tp;
  const S* dsb = reinterpret_cast<const S*>(a.ds) + (((int64_t)bg * a.Tq + t) * a.nslots * nsub * nhg + hg) * 1024;
  // the lane's dQ row (head colh at timestep t); formed where used, not kept live
  auto dq_row = [&]() __attribute__((always_inline)) {
    return reinterpret_cast<S*>(a.dq) + b * a.sdq_b + (int64_t)colh * a.sdq_h + (int64_t)t * a.sdq_t;
  };
  uint4 kf[2][DK / 16];
  auto load = [&](int i, int kc2) __attribute__((always_inline)) {
    const int slot = i / nsub, sub = i - slot * nsub;
    const int key0 = __builtin_amdgcn_readlane(lv, slot) * a.lprime + sub * 64;
#pragma unroll
    for (int j = 0; j < DK / 16; ++j) kf[kc2][j] = ld_colfrag<T>(kcf, key0 / 32 + kc2, j, DK, lane);
  };
  // buffer q & 1 receives batch q's dS fragments, or, for the first q past the last
  // tile, the dQ rows (copy k, lane L: head L % 16, 16-byte piece 4k + L / 16 of its
  // row).  The copies are invisible to the compiler's wait insertion; every K^T load of
  // a batch's tiles is issued after the batch's copies, so the waits for those loads
  // (loads complete in issue order) cover them.
  const int nbatch = (nt + kDsBatch - 1) / kDsBatch;
  auto stage = [&](int q) __attribute__((always_inline)) {
    if (q < nbatch) {
#pragma unroll
      for (int u = 0; u < kDsBatch; ++u) {
        const int i = min(q * kDsBatch + u, nt - 1);
#pragma unroll
        for (int kc2 = 0; kc2 < 2; ++kc2)
          copy16_to_lds_async(dsb + (int64_t)i * nhg * 1024 + (kc2 * 64 + lane) * EPF, &s_ds[wave][q & 1][u * 2 + kc2][0]);
      }
    } else if (q == nbatch && acc_lds) {
      // one opaque base, so the compiler does not keep every copy's address live
      // through the tile loop
      uintptr_t src = reinterpret_cast<uintptr_t>(dq_row() + g4 * 8);
      asm volatile("" : "+v"(src));
#pragma unroll
      for (int k = 0; k < DK / 32; ++k) copy16_to_lds_async(reinterpret_cast<const S*>(src) + 32 * k, &s_ds[wave][q & 1][k][0]);
    }
  };
  f32x4 dqa[DK / 16];
#pragma unroll
  for (int j = 0; j < DK / 16; ++j) dqa[j] = zero4();
  stage(0);
  stage(1);
  if (nt > 0) {
    __builtin_amdgcn_sched_barrier(0);
    load(0, 0);
    __builtin_amdgcn_sched_barrier(0);
    load(0, 1);
    __builtin_amdgcn_sched_barrier(0);
  }
  int q = 0, u = 0;  // tile i = q * kDsBatch + u
  for (int i = 0; i < nt; ++i) {
    const int nx = i + 1 < nt ? i + 1 : i;  // unconditional loads (the last tile re-reads itself)
    // a new batch starts: the buffer of the batch before it is free (its fragments were
    // read in that batch's last tile), so the next stage goes out now
    if (u == 0 && q > 0) stage(q + 1);
#pragma unroll
    for (int kc2 = 0; kc2 < 2; ++kc2) {
      // the wait for this chunk's K^T fragments also covers its dS copy
      asm volatile("" ::"v"(kf[kc2][DK / 16 - 1].x) : "memory");
      const uint4 df = s_ds[wave][q & 1][u * 2 + kc2][lane];
#pragma unroll
      for (int j = 0; j < DK / 16; ++j) dqa[j] = Mma<T>::run(dqa[j], kf[kc2][j], df);
      // keep the order: this chunk's products, then the next tile's loads into its
      // registers (the scheduler would otherwise hoist the loads and wait for all of them)
      __builtin_amdgcn_sched_barrier(0);
      load(nx, kc2);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (++u == kDsBatch) { u = 0; ++q; }
  }
  // every copy has landed (and none still writes this workgroup's LDS when it ends)
  wait_vmcnt<0>();
  asm volatile("" ::: "memory");
  const char* acc = reinterpret_cast<const char*>(&s_ds[wave][nbatch & 1][0][0]);
  S* dqp = dq_row();
#pragma unroll
  for (int j = 0; j < DK / 16; ++j) {
    f32x4 v = dqa[j] * a.scale;
    if (a.dq_acc) {
      // the caller's running dQ sum: columns 16 j + 4 g4 .. + 3 of head c16 (8 bytes)
      const int p = 2 * j + (g4 >> 1);  // the 16-byte piece of the row
      const uint2 r = *reinterpret_cast<const uint2*>(acc + (p >> 2) * 1024 + ((p & 3) * 16 + c16) * 16 + 8 * (g4 & 1));
      v += raw4_f32(r);
    }
    store4<T>(dqp + j * 16 + 4 * g4, v);
  }
}

template <typename T, int DK, int DV>
void launch_attn_sel_dq(const AttnArgs& a, hipStream_t s) {
  if constexpr (sizeof(typename Store<T>::type) == 2) {
    if (a.ds) {
      const int nwaves = a.B * a.G * a.Tq * (a.hpg / 16);
      // the dQ rows go through LDS (16-byte pieces: the entry points accept only dQ rows
      // that start 16-byte aligned)
      const int acc_lds = a.dq_acc;
      hipLaunchKernelGGL((attn_sel_dq_ds_kernel<T, DK>), dim3((nwaves + 3) / 4), dim3(256), 0, s, a, nwaves, acc_lds);
      return;
    }
  }
  const int ncoltiles = (a.Tq * a.hpg + 63) / 64;
  hipLaunchKernelGGL((attn_sel_dq_kernel<T, DK, DV>), dim3(ncoltiles * a.B * a.G), dim3(256), 0, s, a, ncoltiles);
}

}  // namespace nsa
