// Forward attention for the three NSA branches (sliding window, compression,
// top-n selection) on gfx950.
//
// One workgroup = kFwdWaves waves = kFwdCols query columns of one (batch, KV group).  A
// column is one (timestep, head) pair of the group, flattened time-major, so the
// whole group's heads at a timestep share every K/V tile that is staged in LDS
// (one K/V load per GQA group instead of one per head).
//
// The product is computed transposed: S^T[key, col] = K[key,:] . Q[col,:], so that
// the accumulator tile lands with one column per lane.  The online-softmax row
// statistics (running max m and sum l) are then per-lane scalars, and the
// probability tile P^T feeds O^T[dv, col] += V^T[dv, key] P^T[key, col] directly as
// the MFMA B operand (see nsa_device.h for the fragment conventions).
//
// Key sets per branch (reference semantics: nsa/reference.py:13-78, :81-147,
// :205-254):
//   sliding     key j visible to query t iff  t - window < j <= t
//   compression key i visible iff block_ends[i] <= t  (no visible key -> out 0)
//   selection   key j visible iff j <= t and j lies in one of the row's selected
//               blocks [idx*l', idx*l'+l') (union, so a repeated index counts once)
#pragma once
#include <algorithm>
#include "nsa_attn.h"
#include "nsa_device.h"
#include "nsa_attn_sel.h"

namespace nsa {

// Workgroup = kFwdWaves waves x kFwdNSub subtiles x 16 columns.  The K and V^T
// fragments of a 64-key tile are copied from the fragment-native krf / vcf layouts
// (each fragment one contiguous 1 KB run) to LDS by the direct-to-LDS loads
// (global_load_lds_dwordx4: lane l's 16 bytes land at base + 16 l), one fragment per
// instruction, into a double buffer: the copy of tile i+1 is in flight
// while tile i is used, no register holds staging data, and each fragment read is a
// conflict-free 16-byte-per-lane LDS read.  Every fragment read feeds the products of
// all NSUB subtiles of the wave.
template <typename T, int DK, int DV>
struct FwdTile {
  static constexpr int KC = Elem<T>::kKChunk;
  static constexpr int CK = CFrag<T>::kKeys;
  static constexpr int NKF = 4 * (DK / KC);          // K fragments (ks, kc)
  static constexpr int NVF = (64 / CK) * (DV / 16);  // V^T fragments (kc2, j)
  static constexpr int BYTES = (NKF + NVF) * 1024;
  // two 8-wave workgroups per CU (four waves per SIMD), so one workgroup's prologue and
  // epilogue overlap the other's tile loop: a double buffer when two workgroups' stages
  // fit the 160 KB of LDS, else one stage (the other workgroup covers the refill)
  static constexpr int NBUF = 2 * BYTES <= 76 * 1024 ? 2 : 1;
  // when two whole stages do not fit: one K region and two V regions, so that the next
  // tile's V copy overlaps this tile's products and its K copy this tile's softmax and P V
  static constexpr bool SPLIT = NBUF == 1 && 2 * (NKF + 2 * NVF) * 1024 <= 152 * 1024;
  static constexpr int LDS = NBUF == 2 ? 2 * BYTES : SPLIT ? (NKF + 2 * NVF) * 1024 : BYTES;
};

template <typename T, int DK, int DV, int BR>
__global__ __launch_bounds__(64 * kFwdWaves) void attn_fwd_kernel(AttnArgs a) {
  static_assert(BR == kSliding || BR == kCompression, "selection uses attn_sel_fwd_kernel");
  using S = typename Store<T>::type;
  using FT = FwdTile<T, DK, DV>;
  constexpr int EPF = Elem<T>::kPerFrag;
  constexpr int KC = Elem<T>::kKChunk;
  constexpr int NKC = DK / KC;
  constexpr int NSUB = kFwdNSub;
  constexpr int CK = CFrag<T>::kKeys;
  constexpr int CT = CK / 16;
  constexpr int NW = kFwdWaves;
  static_assert(DK % KC == 0 && DV % 16 == 0, "head dims");

  extern __shared__ __attribute__((aligned(16))) uint4 fwd_lds[];  // [NBUF][NKF + NVF][64] or [NKF + 2 NVF][64]
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
  const int col_base = blockIdx.x * kFwdCols;
  // positions are absolute (query row r is at a.q0 + r); rows are addressed relatively
  const int t_first = col_base / hpg + a.q0;
  const int t_last = min(a.Tq - 1, (col_base + kFwdCols - 1) / hpg) + a.q0;
  const float scale2 = a.scale * kLog2e;

  const S* qbase = reinterpret_cast<const S*>(a.q);
  const S* krf = reinterpret_cast<const S*>(a.krf) + (int64_t)bg * a.Tp * DK;
  const S* vcf = reinterpret_cast<const S*>(a.vcf) + (int64_t)bg * DV * a.Tp;

  // ---- per-lane column state -------------------------------------------------
  int colt[NSUB];
  int colh[NSUB];
  bool colv[NSUB];
  int sub_t0[NSUB], sub_t1[NSUB];
  bool f0_full[NSUB];
  uint4 qf[NSUB][NKC];
#pragma unroll
  for (int s = 0; s < NSUB; ++s) {
    const int f0 = col_base + (wave * NSUB + s) * 16;
    const int f = f0 + c16;
    f0_full[s] = f0 + 16 <= ncols;
    colv[s] = f < ncols;
    colt[s] = colv[s] ? f / hpg : 0;
    colh[s] = colv[s] ? grp * hpg + f % hpg : 0;
    sub_t0[s] = f0 / hpg + a.q0;
    sub_t1[s] = f0 < ncols ? min(a.Tq - 1, (f0 + 15) / hpg) + a.q0 : -1;
    const S* qp = qbase + b * a.sq_b + (int64_t)colh[s] * a.sq_h + (int64_t)colt[s] * a.sq_t;
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc)
      qf[s][kc] = colv[s] ? *reinterpret_cast<const uint4*>(qp + kc * KC + g4 * EPF) : make_uint4(0, 0, 0, 0);
  }

  f32x4 oacc[NSUB][DV / 16];
  float m2[NSUB], mtrue[NSUB], lsum[NSUB];  // exponent reference, true maximum, sum
  // bf16: the column sums of P come from the matrix cores (the packed P fragment times an
  // all-ones A operand: every row of the 16x16 result holds the column's sum of the bf16
  // probabilities, the same rounded values the P.V product uses) instead of per-element
  // adds and lane reductions; the exponent argument is a single fma
  constexpr bool kMmaSum = sizeof(S) == 2;
  f32x4 lacc[NSUB];
  const uint4 ones = make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
#pragma unroll
  for (int s = 0; s < NSUB; ++s) {
    m2[s] = -INFINITY;
    mtrue[s] = -INFINITY;
    lsum[s] = 0.f;
    lacc[s] = zero4();
#pragma unroll
    for (int j = 0; j < DV / 16; ++j) oacc[s][j] = zero4();
  }

  // ---- tile list ---------------------------------------------------------------
  int ntiles = 0;
  int key_lo = 0;
  if (BR == kSliding) {
    key_lo = max(0, t_first - a.window + 1) & ~31;  // 32-key aligned (C-permuted V^T chunks)
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

  // ---- direct-to-LDS copies of fragments [f0, f1) of one tile (K rowfrags first, then
  // V^T colfrags) to dst: wave w copies fragments f0 + w, f0 + w + NW, ...; async: the
  // in-loop copies, hidden from the compiler's wait insertion (the loop waits for them
  // itself before its barrier) ----
  auto copy_frags = [&](int key0, uint4* dst, int f0, int f1, auto async) __attribute__((always_inline)) {
    for (int f = f0 + wave; f < f1; f += NW) {
      const S* src;
      if (f < FT::NKF) {  // K rowfrag (16-key group (key0 >> 4) + ks, feature chunk kc)
        const int ks = f / NKC, kc = f % NKC;
        src = krf + ((((int64_t)(key0 >> 4) + ks) * NKC + kc) * 64 + lane) * EPF;
      } else {  // V^T colfrag (key chunk key0 / CK + kc2, feature group j)
        const int v = f - FT::NKF, kc2 = v / (DV / 16), j = v % (DV / 16);
        src = vcf + ((((int64_t)(key0 / CK) + kc2) * (DV / 16) + j) * 64 + lane) * EPF;
      }
      if constexpr (decltype(async)::value) copy16_to_lds_async(src, dst + (f - f0) * 64);
      else copy16_to_lds(src, dst + (f - f0) * 64);
    }
  };
  auto copy_tile = [&](int key0, int buf, auto async) __attribute__((always_inline)) {
    copy_frags(key0, fwd_lds + buf * (FT::NKF + FT::NVF) * 64, 0, FT::NKF + FT::NVF, async);
  };
  auto tile_key0 = [&](int it) -> int { return BR == kSliding ? key_lo + it * 64 : it * 64; };
  int pbe = 0x7fffffff;
  auto load_be = [&](int key0) {
    if (BR == kCompression && tid < 64) {
      const int key = key0 + tid;
      pbe = key < a.Tkv ? a.block_ends[key] : 0x7fffffff;
    }
  };
  // S^T for every subtile: each K fragment read from LDS feeds NSUB products
  auto compute_s = [&](f32x4 (&st)[NSUB][4], const uint4* kb) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int s = 0; s < NSUB; ++s) st[s][ks] = zero4();
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc) {
        const uint4 kf = kb[(ks * NKC + kc) * 64 + lane];
#pragma unroll
        for (int s = 0; s < NSUB; ++s) st[s][ks] = Mma<T>::run(st[s][ks], kf, qf[s][kc]);
      }
    }
  };
  // masking, online softmax and O^T += V^T P^T for the tile at key0 in stage buf
  auto softmax_pv = [&](f32x4 (&st)[NSUB][4], int key0, const uint4* vb, const int* sbe) __attribute__((always_inline)) {
    int be_max = 0;
    if (BR == kCompression) {
      be_max = wave_butterfly(sbe[lane], [](int x, int y) { return max(x, y); });
    }
    uint4 pf[NSUB][64 / CK];
#pragma unroll
    for (int s = 0; s < NSUB; ++s) {
      const int t = colt[s] + a.q0;  // absolute position
      // sliding: the column sees keys [kmin_s, kmin_s + kspan_s) (branch-free test)
      const int kmin_s = max(t - a.window + 1, 0);
      const uint32_t kspan_s = colv[s] ? (uint32_t)max(0, min(t, a.Tkv - 1) + 1 - kmin_s) : 0u;
      // interior tiles (every key visible to every column of the subtile) skip masking
      bool all_visible = false;
      if (BR == kSliding)
        all_visible = f0_full[s] && key0 + 63 <= sub_t0[s] && key0 > sub_t1[s] - a.window && key0 + 63 < a.Tkv;
      else if (BR == kCompression)
        all_visible = f0_full[s] && be_max <= sub_t0[s];
      // the maximum is taken over the raw products (scale2 > 0 commutes with max); the
      // exponent argument is the rounded product minus the reference (not one fma), so
      // the column maximum maps to exp2(0) = 1 exactly
      float mx = -INFINITY;
      if (all_visible) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
          for (int i = 0; i < 4; ++i) mx = fmaxf(mx, st[s][ks][i]);
      } else {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = key0 + ks * 16 + 4 * g4 + i;
            bool ok;
            if (BR == kSliding) ok = (uint32_t)(key - kmin_s) < kspan_s;
            else ok = colv[s] & (sbe[ks * 16 + 4 * g4 + i] <= t);
            const float v = ok ? st[s][ks][i] : -INFINITY;
            st[s][ks][i] = v;
            mx = fmaxf(mx, v);
          }
        }
      }
      mx = wave_max16(mx) * scale2;
      mtrue[s] = fmaxf(mtrue[s], mx);
      // lazy rescale: the exponent reference m2 moves only when some column's maximum
      // exceeds it by more than kLazyRescale (p <= 2^kLazyRescale meanwhile); the true
      // maximum is tracked for M and the final sum is brought to it in the epilogue
      if (__ballot(mx > m2[s] + kLazyRescale) != 0ull) {
        const float mnew = fmaxf(m2[s], mtrue[s]);
        const float alpha = m2[s] == -INFINITY ? 0.f : fast_exp2(m2[s] - mnew);
        lsum[s] *= alpha;
        lacc[s] *= alpha;
#pragma unroll
        for (int j = 0; j < DV / 16; ++j) oacc[s][j] *= alpha;
        m2[s] = mnew;
      }
      const float nref = m2[s] == -INFINITY ? 0.f : -m2[s];
      if constexpr (kMmaSum) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
          for (int i = 0; i < 4; ++i) st[s][ks][i] = fast_exp2(fmaf(st[s][ks][i], scale2, nref));
      } else {
        float rs = 0.f;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p = fast_exp2(mul_add_rounded(st[s][ks][i], scale2, nref));
            st[s][ks][i] = p;
            rs += p;
          }
        }
        rs = wave_sum16(rs);
        lsum[s] += rs;
      }
#pragma unroll
      for (int kc2 = 0; kc2 < 64 / CK; ++kc2) pf[s][kc2] = CFrag<T>::pack(st[s][kc2 * CT], st[s][kc2 * CT + CT - 1]);
    }

    // O^T += V^T P^T: each V^T fragment read from LDS feeds NSUB products
#pragma unroll
    for (int kc2 = 0; kc2 < 64 / CK; ++kc2) {
#pragma unroll
      for (int j = 0; j < DV / 16; ++j) {
        const uint4 vf = vb[(kc2 * (DV / 16) + j) * 64 + lane];
#pragma unroll
        for (int s = 0; s < NSUB; ++s) oacc[s][j] = Mma<T>::run(oacc[s][j], vf, pf[s][kc2]);
      }
      if constexpr (kMmaSum) {
#pragma unroll
        for (int s = 0; s < NSUB; ++s) lacc[s] = Mma<T>::run(lacc[s], ones, pf[s][kc2]);
      }
    }
  };

  f32x4 st[NSUB][4];
  if constexpr (FT::SPLIT) {
    // [K][V0][V1]: tile it's V in region it & 1.  The next tile's V is copied at the top
    // (its region held tile it-1's V, which every wave is past), its K once every wave's
    // S^T products have read this tile's K.
    uint4* kreg = fwd_lds;
    auto vreg = [&](int vb) { return fwd_lds + (FT::NKF + vb * FT::NVF) * 64; };
    if (ntiles > 0) {
      copy_frags(tile_key0(0), kreg, 0, FT::NKF, std::false_type{});
      copy_frags(tile_key0(0), vreg(0), FT::NKF, FT::NKF + FT::NVF, std::false_type{});
      load_be(tile_key0(0));
    }
    for (int it = 0; it < ntiles; ++it) {
      const int vb = it & 1;
      if (BR == kCompression && tid < 64) s_be[it & 1][tid] = pbe;
      __builtin_amdgcn_s_waitcnt(0);  // this wave's copies of tile it have landed
      __syncthreads();                // every wave's have; tile it-1 is no longer read
      if (it + 1 < ntiles) {
        copy_frags(tile_key0(it + 1), vreg(vb ^ 1), FT::NKF, FT::NKF + FT::NVF, std::true_type{});
        load_be(tile_key0(it + 1));
      }
      compute_s(st, kreg);
      if (it + 1 < ntiles) {
        __syncthreads();  // every wave's S^T products have read this tile's K
        copy_frags(tile_key0(it + 1), kreg, 0, FT::NKF, std::true_type{});
      }
      softmax_pv(st, tile_key0(it), vreg(vb), s_be[it & 1]);
    }
  } else {
    if (ntiles > 0) {
      copy_tile(tile_key0(0), 0, std::false_type{});
      load_be(tile_key0(0));
    }
    for (int it = 0; it < ntiles; ++it) {
      const int buf = FT::NBUF == 2 ? (it & 1) : 0;
      if (BR == kCompression && tid < 64) s_be[it & 1][tid] = pbe;
      __builtin_amdgcn_s_waitcnt(0);  // this wave's copies of tile it have landed
      __syncthreads();                // every wave's have; tile it-1 is no longer read
      if (FT::NBUF == 2 && it + 1 < ntiles) {
        copy_tile(tile_key0(it + 1), buf ^ 1, std::true_type{});
        load_be(tile_key0(it + 1));
      }
      const uint4* kb = fwd_lds + buf * (FT::NKF + FT::NVF) * 64;
      compute_s(st, kb);
      softmax_pv(st, tile_key0(it), kb + FT::NKF * 64, s_be[it & 1]);
      if (FT::NBUF == 1 && it + 1 < ntiles) {  // single buffer: refill once every wave is done
        __syncthreads();
        copy_tile(tile_key0(it + 1), 0, std::true_type{});
        load_be(tile_key0(it + 1));
      }
    }
  }

  // ---- epilogue: normalise, store O, L = log(l), M = max s -----------------------
  // bf16: the workgroup's output rows are staged in LDS (free once every wave is past the
  // tile loop) and stored as 16-byte row pieces, 16 lanes per 256-byte row, together with
  // the gated mix when asked; fp32 stores from the accumulator lanes.
  constexpr bool kStage = sizeof(S) == 2;
  constexpr int DVP = DV + 8;  // staged row pitch (elements): 16-byte pad against bank conflicts
  S* obase = reinterpret_cast<S*>(a.o);
  S* stage = reinterpret_cast<S*>(fwd_lds);
  // bf16 with the gated mix: each thread's pieces of the two other branch outputs and
  // the gates are requested here, before the normalise and staging below, so their HBM
  // round trip overlaps that work instead of following it piece by piece
  constexpr int PPR = DV / EPF;  // 16-byte pieces per row
  constexpr int NPC = (kFwdCols * PPR + 64 * NW - 1) / (64 * NW);  // pieces per thread
  uint4 mx0[kStage ? NPC : 1], mx1[kStage ? NPC : 1];
  float mg[kStage ? NPC : 1][3];
  const int nrow = min(kFwdCols, ncols - col_base);
  const IntDiv hdiv = IntDiv::make(hpg);
  const int64_t bht = (int64_t)a.B * a.H * a.Tq;
  if constexpr (kStage) {
    if (a.mix_out) {
#pragma unroll
      for (int i = 0; i < NPC; ++i) {
        const int p = tid + i * 64 * NW;
        if (p < nrow * PPR) {
          const int cl = p / PPR, e = (p % PPR) * EPF;
          const int f = col_base + cl;
          const int t = hdiv.div(f), h = grp * hpg + hdiv.mod(f);
          const int64_t ooff = b * a.so_b + (int64_t)h * a.so_h + (int64_t)t * a.so_t;
          const int64_t srow = ((int64_t)b * a.H + h) * a.Tq + t;
          mx0[i] = *reinterpret_cast<const uint4*>(reinterpret_cast<const S*>(a.mix_o0) + ooff + e);
          mx1[i] = *reinterpret_cast<const uint4*>(reinterpret_cast<const S*>(a.mix_o1) + ooff + e);
          mg[i][0] = a.mix_gates[srow];
          mg[i][1] = a.mix_gates[bht + srow];
          mg[i][2] = a.mix_gates[2 * bht + srow];
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int s = 0; s < NSUB; ++s) {
    if (!colv[s]) continue;
    if constexpr (kMmaSum) lsum[s] = lacc[s][0];
    const float inv = lsum[s] > 0.f ? 1.f / lsum[s] : 0.f;
    // the sum relative to the true maximum (m2 <= mtrue, equal when both are -inf)
    if (lsum[s] > 0.f) lsum[s] *= fast_exp2(m2[s] - mtrue[s]);
    if constexpr (kStage) {
      S* row = stage + ((wave * NSUB + s) * 16 + c16) * DVP;
#pragma unroll
      for (int j = 0; j < DV / 16; ++j) store4<T>(row + j * 16 + 4 * g4, oacc[s][j] * inv);
    } else {
      const int64_t ooff = b * a.so_b + (int64_t)colh[s] * a.so_h + (int64_t)colt[s] * a.so_t;
#pragma unroll
      for (int j = 0; j < DV / 16; ++j) store4<T>(obase + ooff + j * 16 + 4 * g4, oacc[s][j] * inv);
      if (a.mix_out) {
        // gated mix of the three branch outputs as stored: g0 o_0 + g1 o_1 + g2 o,
        // summed in fp32 and rounded once
        const int64_t srow = ((int64_t)b * a.H + colh[s]) * a.Tq + colt[s];
        const float g0 = a.mix_gates[srow], g1 = a.mix_gates[bht + srow], g2 = a.mix_gates[2 * bht + srow];
        const S* o0 = reinterpret_cast<const S*>(a.mix_o0) + ooff;
        const S* o1 = reinterpret_cast<const S*>(a.mix_o1) + ooff;
        S* xp = reinterpret_cast<S*>(a.mix_out) + b * a.smx_b + (int64_t)colh[s] * a.smx_h +
                (int64_t)colt[s] * a.smx_t;
#pragma unroll
        for (int j = 0; j < DV / 16; ++j) {
          const int e = j * 16 + 4 * g4;
          const f32x4 own = oacc[s][j] * inv;
          const f32x4 x0 = load4<T>(o0 + e), x1 = load4<T>(o1 + e);
          f32x4 m;
#pragma unroll
          for (int u = 0; u < 4; ++u) m[u] = g0 * x0[u] + g1 * x1[u] + g2 * own[u];
          store4<T>(xp + e, m);
        }
      }
    }
    if (g4 == 0) {
      if (a.L)
        a.L[b * a.sl_b + (int64_t)colh[s] * a.sl_h + (int64_t)colt[s] * a.sl_t] =
            lsum[s] > 0.f ? logf(lsum[s]) : -INFINITY;
      if (a.M)
        a.M[b * a.sm_b + (int64_t)colh[s] * a.sm_h + (int64_t)colt[s] * a.sm_t] = mtrue[s] * kLn2;
    }
  }
  if constexpr (kStage) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NPC; ++i) {
      const int p = tid + i * 64 * NW;
      if (p >= nrow * PPR) break;
      const int cl = p / PPR, e = (p % PPR) * EPF;
      const int f = col_base + cl;
      const int t = hdiv.div(f), h = grp * hpg + hdiv.mod(f);
      const uint4 v = *reinterpret_cast<const uint4*>(stage + cl * DVP + e);
      const int64_t ooff = b * a.so_b + (int64_t)h * a.so_h + (int64_t)t * a.so_t;
      *reinterpret_cast<uint4*>(obase + ooff + e) = v;
      if (a.mix_out) {
        // gated mix of the three branch outputs as stored: g0 o_0 + g1 o_1 + g2 o,
        // summed in fp32 and rounded once
        const float g0 = mg[i][0], g1 = mg[i][1], g2 = mg[i][2];
        const uint32_t w0[4] = {mx0[i].x, mx0[i].y, mx0[i].z, mx0[i].w};
        const uint32_t w1[4] = {mx1[i].x, mx1[i].y, mx1[i].z, mx1[i].w};
        const uint32_t w2[4] = {v.x, v.y, v.z, v.w};
        uint32_t r[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float lo = g0 * __uint_as_float(w0[k] << 16) + g1 * __uint_as_float(w1[k] << 16) +
                           g2 * __uint_as_float(w2[k] << 16);
          const float hi = g0 * __uint_as_float(w0[k] & 0xffff0000u) + g1 * __uint_as_float(w1[k] & 0xffff0000u) +
                           g2 * __uint_as_float(w2[k] & 0xffff0000u);
          r[k] = pack_bf16x2(lo, hi);
        }
        S* xp = reinterpret_cast<S*>(a.mix_out) + b * a.smx_b + (int64_t)h * a.smx_h + (int64_t)t * a.smx_t;
        *reinterpret_cast<uint4*>(xp + e) = make_uint4(r[0], r[1], r[2], r[3]);
      }
    }
  }
}

template <typename T, int DK, int DV, int BR>
void launch_attn_fwd(const AttnArgs& a, hipStream_t s) {
  if constexpr (BR == kSelection) {
    launch_attn_sel_fwd<T, DK, DV>(a, s);  // per-wave selection kernel
  } else {
    using FT = FwdTile<T, DK, DV>;
    // the K/V tile stages, reused by the bf16 epilogue for the workgroup's output rows
    const size_t stage = sizeof(typename Store<T>::type) == 2 ? (size_t)kFwdCols * (DV + 8) * 2 : 0;
    const size_t lds = std::max((size_t)FT::LDS, stage);
    allow_dynamic_lds(reinterpret_cast<const void*>(&attn_fwd_kernel<T, DK, DV, BR>), lds);
    dim3 grid((a.Tq * a.hpg + kFwdCols - 1) / kFwdCols, a.B * a.G);
    hipLaunchKernelGGL((attn_fwd_kernel<T, DK, DV, BR>), grid, dim3(64 * kFwdWaves), lds, s, a);
  }
}

}  // namespace nsa
