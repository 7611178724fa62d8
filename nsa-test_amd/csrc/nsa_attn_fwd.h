// Forward attention for the three NSA branches (sliding window, compression,
// top-n selection) on gfx950.
//
// One workgroup = 4 waves = kFwdCols query columns of one (batch, KV group).  A
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
#include "nsa_attn.h"
#include "nsa_device.h"
#include "nsa_attn_sel.h"

namespace nsa {

template <typename T, int DK, int DV, int BR>
__global__ __launch_bounds__(256) void attn_fwd_kernel(AttnArgs a) {
  static_assert(BR == kSliding || BR == kCompression, "selection uses attn_sel_fwd_kernel");
  using S = typename Store<T>::type;
  constexpr int EPF = Elem<T>::kPerFrag;
  constexpr int KC = Elem<T>::kKChunk;
  constexpr int NKC = DK / KC;
  constexpr int NSUB = kFwdNSub;
  constexpr int KP = DK + EPF;  // padded LDS row of the K tile
  constexpr int VP = 64 + EPF;  // padded LDS row of the V^T tile
  constexpr int CK = CFrag<T>::kKeys;
  constexpr int CT = CK / 16;
  static_assert(DK % KC == 0 && DV % 16 == 0, "head dims");

  __shared__ __attribute__((aligned(16))) S Ks[64 * KP];
  __shared__ __attribute__((aligned(16))) S Vs[DV * VP];
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
  const int col_base = blockIdx.x * kFwdCols;
  const int t_first = col_base / hpg;
  const int t_last = min(a.Tq - 1, (col_base + kFwdCols - 1) / hpg);
  const float scale2 = a.scale * kLog2e;

  const S* qbase = reinterpret_cast<const S*>(a.q);
  const S* kt = reinterpret_cast<const S*>(a.kt) + (int64_t)bg * a.Tp * DK;
  const S* vt = reinterpret_cast<const S*>(a.vt) + (int64_t)bg * DV * a.Tp;

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
    sub_t0[s] = f0 / hpg;
    sub_t1[s] = f0 < ncols ? min(a.Tq - 1, (f0 + 15) / hpg) : -1;
    const S* qp = qbase + b * a.sq_b + (int64_t)colh[s] * a.sq_h + (int64_t)colt[s] * a.sq_t;
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc)
      qf[s][kc] = colv[s] ? *reinterpret_cast<const uint4*>(qp + kc * KC + g4 * EPF) : make_uint4(0, 0, 0, 0);
  }

  f32x4 oacc[NSUB][DV / 16];
  float m2[NSUB], lsum[NSUB];
#pragma unroll
  for (int s = 0; s < NSUB; ++s) {
    m2[s] = -INFINITY;
    lsum[s] = 0.f;
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
    for (int i = tid; i < a.Tkv; i += 256)
      if (a.block_ends[i] <= t_last) mx = i + 1;
    if (mx) atomicMax(&s_misc[0], mx);
    __syncthreads();
    ntiles = (s_misc[0] + 63) / 64;
  }

  // ---- K rows / V^T columns of a 64-key tile: loaded into registers one tile ahead,
  // stored to LDS once the previous tile's products are done ----
  constexpr int NKP = (64 * (DK / EPF) + 255) / 256;
  constexpr int NVP = (DV * (64 / EPF) + 255) / 256;
  u32x4 pk[NKP], pv[NVP];
  int pbe = 0x7fffffff;
  auto tile_key0 = [&](int it) -> int { return BR == kSliding ? key_lo + it * 64 : it * 64; };
  auto load_tile = [&](int key0) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NKP; ++j) {
      const int c = min(tid + 256 * j, 64 * (DK / EPF) - 1);
      pk[j] = *reinterpret_cast<const u32x4*>(kt + (int64_t)(key0 + c / (DK / EPF)) * DK + (c % (DK / EPF)) * EPF);
    }
#pragma unroll
    for (int j = 0; j < NVP; ++j) {
      const int c = min(tid + 256 * j, DV * (64 / EPF) - 1);
      pv[j] = *reinterpret_cast<const u32x4*>(vt + (int64_t)(c / (64 / EPF)) * a.Tp + key0 + (c % (64 / EPF)) * EPF);
    }
    if (BR == kCompression && tid < 64) {
      const int key = key0 + tid;
      pbe = key < a.Tkv ? a.block_ends[key] : 0x7fffffff;
    }
  };
  if (ntiles > 0) load_tile(tile_key0(0));

  for (int it = 0; it < ntiles; ++it) {
    const int key0 = tile_key0(it);
    // ---- stage K rows and V^T columns of keys [key0, key0+64) ----
#pragma unroll
    for (int j = 0; j < NKP; ++j) {
      const int c = tid + 256 * j;
      if ((64 * (DK / EPF)) % 256 == 0 || c < 64 * (DK / EPF))
        *reinterpret_cast<u32x4*>(&Ks[(c / (DK / EPF)) * KP + (c % (DK / EPF)) * EPF]) = pk[j];
    }
#pragma unroll
    for (int j = 0; j < NVP; ++j) {
      const int c = tid + 256 * j;
      if ((DV * (64 / EPF)) % 256 == 0 || c < DV * (64 / EPF))
        *reinterpret_cast<u32x4*>(&Vs[(c / (64 / EPF)) * VP + (c % (64 / EPF)) * EPF]) = pv[j];
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

#pragma unroll
    for (int s = 0; s < NSUB; ++s) {
      f32x4 st[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        st[ks] = zero4();
        const S* krow = &Ks[(ks * 16 + c16) * KP];
#pragma unroll
        for (int kc = 0; kc < NKC; ++kc) st[ks] = Mma<T>::run(st[ks], frag_std<T>(krow + kc * KC, g4), qf[s][kc]);
      }

      const int t = colt[s];
      // sliding: the column sees keys [kmin_s, kmin_s + kspan_s) (branch-free test)
      const int kmin_s = max(t - a.window + 1, 0);
      const uint32_t kspan_s = colv[s] ? (uint32_t)max(0, min(t, a.Tkv - 1) + 1 - kmin_s) : 0u;
      // interior tiles (every key visible to every column of the subtile) skip masking
      bool all_visible = false;
      if (BR == kSliding)
        all_visible = f0_full[s] && key0 + 63 <= sub_t0[s] && key0 > sub_t1[s] - a.window && key0 + 63 < a.Tkv;
      else if (BR == kCompression)
        all_visible = f0_full[s] && be_max <= sub_t0[s];
      float mx = -INFINITY;
      if (all_visible) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            st[ks][i] *= scale2;
            mx = fmaxf(mx, st[ks][i]);
          }
      } else {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = key0 + ks * 16 + 4 * g4 + i;
            bool ok;
            if (BR == kSliding) ok = (uint32_t)(key - kmin_s) < kspan_s;
            else ok = colv[s] & (s_be[ks * 16 + 4 * g4 + i] <= t);
            const float v = ok ? st[ks][i] * scale2 : -INFINITY;
            st[ks][i] = v;
            mx = fmaxf(mx, v);
          }
        }
      }
      mx = wave_max16(mx);
      const float mnew = fmaxf(m2[s], mx);
      const float mref = mnew == -INFINITY ? 0.f : mnew;
      float rs = 0.f;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = fast_exp2(st[ks][i] - mref);
          st[ks][i] = p;
          rs += p;
        }
      }
      rs = wave_sum16(rs);
      // rescale the running output only when some column's maximum moved
      if (__ballot(mnew > m2[s]) != 0ull) {
        const float alpha = fast_exp2(m2[s] - mref);
        lsum[s] *= alpha;
#pragma unroll
        for (int j = 0; j < DV / 16; ++j) oacc[s][j] *= alpha;
      }
      lsum[s] += rs;
      m2[s] = mnew;

#pragma unroll
      for (int kc2 = 0; kc2 < 64 / CK; ++kc2) {
        const uint4 pf = CFrag<T>::pack(st[kc2 * CT], st[kc2 * CT + CT - 1]);
#pragma unroll
        for (int j = 0; j < DV / 16; ++j) {
          const uint4 vf = frag_cperm<T>(&Vs[(j * 16 + c16) * VP + kc2 * CK], g4);
          oacc[s][j] = Mma<T>::run(oacc[s][j], vf, pf);
        }
      }
    }
    __syncthreads();
  }

  // ---- epilogue: normalise, store O, L = log(l), M = max s -----------------------
  S* obase = reinterpret_cast<S*>(a.o);
#pragma unroll
  for (int s = 0; s < NSUB; ++s) {
    if (!colv[s]) continue;
    const float inv = lsum[s] > 0.f ? 1.f / lsum[s] : 0.f;
    S* op = obase + b * a.so_b + (int64_t)colh[s] * a.so_h + (int64_t)colt[s] * a.so_t;
#pragma unroll
    for (int j = 0; j < DV / 16; ++j) store4<T>(op + j * 16 + 4 * g4, oacc[s][j] * inv);
    if (g4 == 0) {
      if (a.L)
        a.L[b * a.sl_b + (int64_t)colh[s] * a.sl_h + (int64_t)colt[s] * a.sl_t] =
            lsum[s] > 0.f ? logf(lsum[s]) : -INFINITY;
      if (a.M)
        a.M[b * a.sm_b + (int64_t)colh[s] * a.sm_h + (int64_t)colt[s] * a.sm_t] = m2[s] * kLn2;
    }
  }
}

template <typename T, int DK, int DV, int BR>
void launch_attn_fwd(const AttnArgs& a, hipStream_t s) {
  dim3 grid((a.Tq * a.hpg + kFwdCols - 1) / kFwdCols, a.B * a.G);
  if constexpr (BR == kSelection) {
    launch_attn_sel_fwd<T, DK, DV>(a, s);  // per-wave selection kernel
  } else {
    hipLaunchKernelGGL((attn_fwd_kernel<T, DK, DV, BR>), grid, dim3(256), 0, s, a);
  }
}

}  // namespace nsa
