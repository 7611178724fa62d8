// Fused selection scoring on gfx950: Eq. 8 (compressed-attention probabilities),
// Eq. 9 (triangular remap to selection blocks), Eq. 10 (GQA head sum) and the top-n
// with fixed blocks, one workgroup per (batch, group, TT consecutive timesteps).
//
// Nothing is materialised in HBM except the n indices per (b, g, t) (and, when the
// caller asks for them, the p_cmp / p_slc score tensors the reference module returns
// in attn_info).
//
// The fp32 arithmetic follows a fixed order so that the indices are reproducible
// bit for bit (this unit is compiled with -ffp-contract=off):
//   logit   acc = fma(q[e], k[e][i], acc) for e = 0..dk-1, then acc * scale
//   softmax e_i = exp32(s_i - max); sum = 64 lane partials (lane L adds i = L mod 64 in
//           ascending order) combined by xor-butterfly over 32,16,8,4,2,1; p = e / sum
//   Eq. 9   p_slc[j] = sum over (m, n) in the reference's loop order
//           (nsa/kernels.py:1953-1960), starting from 0
//   Eq. 10  heads added in head order (nsa/kernels.py:1990-1993)
//   top-n   the k = min(n, nsel) largest aggregated scores, equal scores ordered by
//           lower block index (the stable descending sort of nsa/kernels.py:2001),
//           then [0, max(0,(t-l')//l'), t//l'] ++ top-k de-duplicated in order,
//           truncated to n, padded with -1 (nsa/kernels.py:2005-2040).
// exp32 is a Cody-Waite reduction plus a degree-7 Taylor polynomial (evaluated with
// fma), flushed to 0 below -64 so no denormal ever enters the pipeline.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "nsa_attn.h"
#include "nsa_device.h"

namespace nsa {

__device__ __forceinline__ float exp32(float x) {
  const float kL2e = 1.44269504088896341f;
  const float kLn2Hi = 0.693145751953125f;
  const float kLn2Lo = 1.42860682030941723212e-6f;
  if (!(x >= -64.0f)) return 0.0f;
  if (x > 0.0f) x = 0.0f;
  const float k = rintf(x * kL2e);
  float r = fmaf(-k, kLn2Hi, x);
  r = fmaf(-k, kLn2Lo, r);
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return p * __uint_as_float((uint32_t)((int)k + 127) << 23);
}

struct ScoreArgs {
  const void* q;
  int64_t sq_b, sq_h, sq_t, sq_d;
  const void* kc;  // compressed keys, element (b, g, e, i)
  int64_t sk_b, sk_g, sk_d, sk_i;
  const int* block_ends;
  int64_t* out;
  int64_t so_b, so_g, so_t, so_n;
  float* p_cmp;  // optional [B,H,T,NB]
  float* p_slc;  // optional [B,H,T,nsel]
  int B, H, G, hpg, T, dk, NB;
  float scale;
  int a, s, nsel, lprime, n, include_fixed;
  int TT;  // timesteps per workgroup
};

constexpr int kMaxRows = 64;  // rows (timestep, head) of one workgroup
constexpr int kMaxCols = 4096;  // compressed blocks a row can score

template <typename S>
__device__ __forceinline__ void unpack16(const uint4& raw, float* v);
template <> __device__ __forceinline__ void unpack16<float>(const uint4& raw, float* v) {
  v[0] = __uint_as_float(raw.x);
  v[1] = __uint_as_float(raw.y);
  v[2] = __uint_as_float(raw.z);
  v[3] = __uint_as_float(raw.w);
}
template <> __device__ __forceinline__ void unpack16<uint16_t>(const uint4& raw, float* v) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    v[2 * u] = __uint_as_float(w[u] << 16);
    v[2 * u + 1] = __uint_as_float(w[u] & 0xffff0000u);
  }
}

// One workgroup per (batch, group, TT consecutive timesteps); NW = blockDim / 64 waves.
// Wave w owns the rows r = w + NW * rr (rr < RPW) of the TT * hpg (timestep, head)
// rows, and lane L of a wave owns the compressed blocks i = L + 64 c (c < C): the
// logits, the softmax and Eq. 9 of a row all stay inside the wave that owns it, in
// registers.  The query row of a wave is wave-uniform, so it is read through the scalar
// unit and broadcast to the FMAs; each 16-byte key load feeds RPW * (16 / sizeof(S))
// FMAs.
template <typename S, int RPW, int C>
// Up to 8 column chunks the accumulators fit 80 VGPRs and six waves per SIMD hide the
// scalar-load latency of the query rows; wider rows keep the compiler's default.
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(C * RPW <= 64 && C <= 8 ? 6 : 1))) void score_topn_kernel(ScoreArgs a, const S* __restrict__ qg) {
  extern __shared__ float lds[];
  constexpr int EV = 16 / sizeof(S);
  const int tid = threadIdx.x, lane = tid & 63;
  const int NW = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bg = blockIdx.y, b = bg / a.G, g = bg % a.G;
  const int t0 = blockIdx.x * a.TT;
  const int TT = min(a.TT, a.T - t0);
  const int hpg = a.hpg;
  const int rows = TT * hpg;  // r = tt * hpg + hh
  const int t_last = t0 + TT - 1;
  const int NB = a.NB, nsel = a.nsel, dk = a.dk;
  const int segw = 64 * a.s + a.a;  // columns Eq. 9 reads for 64 consecutive blocks

  float* pseg = lds + wave * segw;                          // [NW][segw]
  float* ps = lds + NW * segw;                              // [rows][nsel]
  float* agg = ps + rows * nsel;                            // [TT][nsel]
  int* top = reinterpret_cast<int*>(agg + a.TT * nsel);     // [TT][64]
  int* chosen = top + a.TT * 64;                            // [TT][64]

  // columns with any visible row (plus block 0 for the no-visible-block rule)
  __shared__ int s_ncomp;
  if (tid == 0) s_ncomp = 0;
  __syncthreads();
  {
    int mx = 0;
    for (int i = tid; i < NB; i += blockDim.x)
      if (a.block_ends[i] <= t_last) mx = i + 1;
    if (mx) atomicMax(&s_ncomp, mx);
  }
  __syncthreads();
  int ncomp = s_ncomp;
  if (ncomp == 0 && NB > 0) ncomp = 1;
  const int nch = (ncomp + 63) >> 6;  // <= C (checked by the launcher)

  int be[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int i = c * 64 + lane;
    be[c] = (c < nch && i < ncomp) ? a.block_ends[i] : 0x7fffffff;
  }

  // ---- Eq. 8 logits: one sequential fma chain over e = 0..dk-1 per (row, block) ----
  float acc[RPW][C];
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr)
#pragma unroll
    for (int c = 0; c < C; ++c) acc[rr][c] = 0.0f;
  const S* kc = reinterpret_cast<const S*>(a.kc) + b * a.sk_b + g * a.sk_g;
  const S* qb = qg + b * a.sq_b;
  const S* kcol[C];  // the lane's compressed-key rows (past the last block: the last one)
#pragma unroll
  for (int c = 0; c < C; ++c) kcol[c] = kc + (int64_t)min(c * 64 + lane, ncomp - 1) * a.sk_i;
  // Chunks are processed CB at a time, each group under a wave-uniform branch around its
  // own pass over the feature axis, so groups past the last visible block cost nothing.
  constexpr int CB = C < 2 ? C : 2;
#pragma unroll
  for (int cb = 0; cb < C; cb += CB) {
    if (cb < nch) {
      for (int e0 = 0; e0 < dk; e0 += EV) {
        float qv[RPW][EV];
#pragma unroll
        for (int rr = 0; rr < RPW; ++rr) {
          const int r = min(wave + NW * rr, rows - 1);
          const int t = t0 + r / hpg, h = g * hpg + r % hpg;
          unpack16<S>(*reinterpret_cast<const uint4*>(qb + (int64_t)h * a.sq_h + (int64_t)t * a.sq_t + e0), qv[rr]);
        }
        uint4 kraw[CB];
#pragma unroll
        for (int c = 0; c < CB; ++c) kraw[c] = *reinterpret_cast<const uint4*>(kcol[cb + c] + e0);
#pragma unroll
        for (int c = 0; c < CB; ++c) {
          float kv[EV];
          unpack16<S>(kraw[c], kv);
#pragma unroll
          for (int rr = 0; rr < RPW; ++rr)
#pragma unroll
            for (int u = 0; u < EV; ++u) acc[rr][cb + c] = fmaf(qv[rr][u], kv[u], acc[rr][cb + c]);
        }
      }
    }
  }

  // ---- per row: softmax (Eq. 8) and Eq. 9, inside the owning wave ----
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const int r = wave + NW * rr;
    if (r >= rows) continue;  // wave-uniform
    const int t = t0 + r / hpg, h = g * hpg + r % hpg;
    float mx = -INFINITY;
    bool anyv = false;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      if (c < nch) {
        acc[rr][c] = acc[rr][c] * a.scale;
        const bool v = be[c] <= t;
        anyv |= v;
        if (v) mx = fmaxf(mx, acc[rr][c]);
      }
    }
    const bool any_row = __ballot(anyv) != 0ull;
    if (!any_row) mx = __shfl(acc[rr][0], 0);  // block 0 made visible
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    // lane partial over its blocks in ascending order, then the xor butterfly
    float part = 0.0f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      if (c < nch) {
        const bool v = be[c] <= t || (!any_row && c == 0 && lane == 0);
        const float e = v ? exp32(acc[rr][c] - mx) : 0.0f;
        acc[rr][c] = e;
        part += e;
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) part = part + __shfl_xor(part, off);
    const float sum = part;
#pragma unroll
    for (int c = 0; c < C; ++c)
      if (c < nch) acc[rr][c] = acc[rr][c] / sum;
    if (a.p_cmp) {
      float* pc = a.p_cmp + (((int64_t)b * a.H + h) * a.T + t) * NB;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const int i = c * 64 + lane;
        if (i < NB) pc[i] = (c < nch && i < ncomp) ? acc[rr][c] : 0.0f;
      }
    }
    // Eq. 9 in the reference's (m, n) order, 64 selection blocks at a time from a
    // per-wave copy of the columns they read
    float* psr = ps + r * nsel;
    for (int j0 = 0; j0 < nsel; j0 += 64) {
      const int lo = j0 * a.s;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const int i = c * 64 + lane;
        if (i >= lo && i < lo + segw) pseg[i - lo] = (c < nch && i < ncomp) ? acc[rr][c] : 0.0f;
      }
      __builtin_amdgcn_s_waitcnt(0);
      __builtin_amdgcn_wave_barrier();
      const int j = j0 + lane;
      if (j < nsel) {
        float s9 = 0.0f;
        for (int m = 0; m < a.s; ++m)
          for (int nn = 0; nn < a.a; ++nn) {
            const int ci = a.s * j + m + nn;
            if (ci < NB) s9 += ci < ncomp ? pseg[ci - lo] : 0.0f;
          }
        psr[j] = s9;
        if (a.p_slc) a.p_slc[(((int64_t)b * a.H + h) * a.T + t) * nsel + j] = s9;
      }
      __builtin_amdgcn_s_waitcnt(0);
      __builtin_amdgcn_wave_barrier();
    }
  }
  __syncthreads();

  // ---- Eq. 10: heads added in head order ----
  for (int x = tid; x < TT * nsel; x += blockDim.x) {
    const int tt = x / nsel, j = x % nsel;
    float ag = 0.0f;
    for (int hh = 0; hh < hpg; ++hh) ag += ps[(tt * hpg + hh) * nsel + j];
    agg[tt * nsel + j] = ag;
  }
  __syncthreads();

  // ---- top-n (one wave per timestep) ----
  const int kk = min(a.n, nsel);
  for (int tt = wave; tt < TT; tt += NW) {
    const int t = t0 + tt;
    float* ag = agg + tt * nsel;
    for (int rk = 0; rk < kk; ++rk) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      for (int j = lane; j < nsel; j += 64) {
        const float v = ag[j];
        if (v > bv || (v == bv && j < bi)) {
          bv = v;
          bi = j;
        }
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (ov > bv || (ov == bv && oi < bi)) {
          bv = ov;
          bi = oi;
        }
      }
      if (lane == 0) {
        top[tt * 64 + rk] = bi;
        ag[bi] = -INFINITY;  // taken
      }
      __builtin_amdgcn_s_waitcnt(0);
      __builtin_amdgcn_wave_barrier();
    }
    if (lane == 0) {
      int64_t* o = a.out + b * a.so_b + g * a.so_g + (int64_t)t * a.so_t;
      int* sel = chosen + tt * 64;
      int no = 0;
      // fixed candidates [0, max(0, (t - l') / l'), t / l'] first
      const int nc = a.include_fixed ? 3 : 0;
      const int c1 = t >= a.lprime ? (t - a.lprime) / a.lprime : 0;
      const int c2 = t / a.lprime;
      for (int c = 0; c < nc + kk && no < a.n; ++c) {
        const int v = c < nc ? (c == 0 ? 0 : c == 1 ? c1 : c2) : top[tt * 64 + c - nc];
        bool dup = false;
        for (int u = 0; u < no; ++u) dup |= sel[u] == v;
        if (!dup) sel[no++] = v;
      }
      for (int u = 0; u < a.n; ++u) o[(int64_t)u * a.so_n] = u < no ? (int64_t)sel[u] : -1;
    }
  }
}

template <typename S, int RPW, int C>
static hipError_t launch_score_k(const ScoreArgs& a, int nw, size_t lds, hipStream_t st) {
  auto fn = score_topn_kernel<S, RPW, C>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)lds);
  if (e != hipSuccess) return e;
  dim3 grid((a.T + a.TT - 1) / a.TT, a.B * a.G);
  hipLaunchKernelGGL(fn, grid, dim3(64 * nw), lds, st, a, reinterpret_cast<const S*>(a.q));
  return hipGetLastError();
}

template <typename S, int RPW>
static hipError_t launch_score_c(const ScoreArgs& a, int nw, int C, size_t lds, hipStream_t st) {
  switch (C) {
    case 1: return launch_score_k<S, RPW, 1>(a, nw, lds, st);
    case 2: return launch_score_k<S, RPW, 2>(a, nw, lds, st);
    case 4: return launch_score_k<S, RPW, 4>(a, nw, lds, st);
    case 8: return launch_score_k<S, RPW, 8>(a, nw, lds, st);
    case 16: if constexpr (RPW <= 8) return launch_score_k<S, RPW, 16>(a, nw, lds, st); break;
    case 32: if constexpr (RPW <= 4) return launch_score_k<S, RPW, 32>(a, nw, lds, st); break;
    case 64: if constexpr (RPW <= 2) return launch_score_k<S, RPW, 64>(a, nw, lds, st); break;
  }
  return hipErrorInvalidValue;
}

template <typename S>
static hipError_t launch_score_r(const ScoreArgs& a, int nw, int RPW, int C, size_t lds, hipStream_t st) {
  switch (RPW) {
    case 1: return launch_score_c<S, 1>(a, nw, C, lds, st);
    case 2: return launch_score_c<S, 2>(a, nw, C, lds, st);
    case 4: return launch_score_c<S, 4>(a, nw, C, lds, st);
    case 8: return launch_score_c<S, 8>(a, nw, C, lds, st);
  }
  return hipErrorInvalidValue;
}

static int pow2_at_least(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

// Picks (waves, timesteps, rows per wave, column chunks) for the shape.  Returns 0 on
// success, 1 when no configuration fits (too many heads or compressed blocks), 2 on a
// HIP launch error.
int launch_score_topn(int dtype, ScoreArgs a, hipStream_t st) {
  constexpr size_t kLdsMax = 160 * 1024;
  if (a.NB > kMaxCols) return 1;
  const int C = pow2_at_least(max(1, (a.NB + 63) / 64));
  // accumulator budget per lane: RPW * C <= 64 preferred, 128 at most
  for (int budget : {64, 128})
    for (int nw : {4, 8})
      for (int TT : {4, 2, 1}) {
        if (TT > 1 && TT * a.hpg > kMaxRows) continue;
        const int rows = TT * a.hpg;
        const int RPW = pow2_at_least((rows + nw - 1) / nw);
        if (RPW > 8 || RPW * C > budget) continue;
        const int segw = 64 * a.s + a.a;
        const size_t lds = 4 * ((size_t)nw * segw + (size_t)rows * a.nsel + (size_t)TT * a.nsel + (size_t)TT * 128);
        if (lds > kLdsMax) continue;
        a.TT = TT;
        hipError_t e = dtype == kF32 ? launch_score_r<float>(a, nw, RPW, C, lds, st)
                                     : launch_score_r<uint16_t>(a, nw, RPW, C, lds, st);
        return e == hipSuccess ? 0 : 2;
      }
  return 1;
}

}  // namespace nsa

// ------------------------------------------------------------------ C ABI ----
#include "../../include/nsa_hip.h"

#include "nsa_kernels.h"

extern "C" size_t nsa_score_topn_workspace_size(int, int, int, int, int, int, int) { return 0; }

extern "C" int nsa_score_topn(const void* q, const void* k_cmp, const int32_t* block_ends, int64_t* out_idx,
                              float* p_cmp, float* p_slc, int64_t stride_qz, int64_t stride_qh, int64_t stride_qm,
                              int64_t stride_qk, int64_t stride_kz, int64_t stride_kg, int64_t stride_kk,
                              int64_t stride_kn, int64_t stride_iz, int64_t stride_ig, int64_t stride_im,
                              int64_t stride_in, int Z, int H, int n_kv_groups, int n_ctx, int head_dim_qk,
                              int n_blocks, int l, int d, int l_prime, int n, int include_fixed, int n_fixed,
                              int dtype, float scale, void* workspace, size_t workspace_bytes, nsa_stream_t stream) {
  using namespace nsa;
  (void)workspace;
  (void)workspace_bytes;
  if (dtype != NSA_F32 && dtype != NSA_BF16) return nsa::set_error(NSA_ERR_INVALID, "dtype not supported");
  if (Z <= 0 || H <= 0 || n_kv_groups <= 0 || H % n_kv_groups || n_ctx < 0 || head_dim_qk <= 0 || n_blocks < 0)
    return nsa::set_error(NSA_ERR_INVALID, "bad shape");
  if (d <= 0 || l <= 0 || l_prime <= 0 || l % d || l_prime % d)
    return nsa::set_error(NSA_ERR_INVALID, "need l % d == 0 and l_prime % d == 0");
  if (n < 0 || n > 64) return nsa::set_error(NSA_ERR_INVALID, "n outside [0, 64]");
  {
    const int esz = dtype == NSA_F32 ? 4 : 2;
    // strides of size-1 axes never address memory and are not checked
    const bool ok = stride_kk == 1 && (head_dim_qk * esz) % 16 == 0 && ((uintptr_t)k_cmp) % 16 == 0 &&
                    (Z == 1 || (stride_kz * esz) % 16 == 0) && (n_kv_groups == 1 || (stride_kg * esz) % 16 == 0) &&
                    (n_blocks == 1 || (stride_kn * esz) % 16 == 0);
    if (!ok)
      return nsa::set_error(NSA_ERR_LAYOUT,
                            "k_cmp needs a unit-stride feature axis (the [Z,G,N,dk] storage of the reference's "
                            "[Z,G,dk,N] view) with 16-byte aligned rows");
    const bool qok = stride_qk == 1 && ((uintptr_t)q) % 16 == 0 && (Z == 1 || (stride_qz * esz) % 16 == 0) &&
                     (H == 1 || (stride_qh * esz) % 16 == 0) && (n_ctx == 1 || (stride_qm * esz) % 16 == 0);
    if (!qok) return nsa::set_error(NSA_ERR_LAYOUT, "q needs a unit-stride feature axis with 16-byte aligned rows");
  }
  if (n_ctx == 0) return NSA_OK;
  ScoreArgs a{};
  a.q = q;
  a.sq_b = stride_qz;
  a.sq_h = stride_qh;
  a.sq_t = stride_qm;
  a.sq_d = stride_qk;
  a.kc = k_cmp;
  a.sk_b = stride_kz;
  a.sk_g = stride_kg;
  a.sk_d = stride_kk;
  a.sk_i = stride_kn;
  a.block_ends = block_ends;
  a.out = out_idx;
  a.so_b = stride_iz;
  a.so_g = stride_ig;
  a.so_t = stride_im;
  a.so_n = stride_in;
  a.p_cmp = p_cmp;
  a.p_slc = p_slc;
  a.B = Z;
  a.H = H;
  a.G = n_kv_groups;
  a.hpg = H / n_kv_groups;
  a.T = n_ctx;
  a.dk = head_dim_qk;
  a.NB = n_blocks;
  a.scale = scale;
  a.a = l / d;
  a.s = l_prime / d;
  a.nsel = (n_blocks + a.s - 1) / a.s;
  a.lprime = l_prime;
  a.n = n;
  a.include_fixed = include_fixed && n_fixed > 0;
  if (a.hpg > kMaxRows) return nsa::set_error(NSA_ERR_UNSUPPORTED, "more than 64 heads per group");
  int rc;
  {
    TimingScope ts(kIdScore, (hipStream_t)stream);
    rc = launch_score_topn(dtype, a, (hipStream_t)stream);
  }
  if (rc == 1) {
    char msg[128];
    snprintf(msg, sizeof(msg), "no scoring configuration for %d heads per group and %d compressed blocks", a.hpg,
             a.NB);
    return nsa::set_error(NSA_ERR_UNSUPPORTED, msg);
  }
  if (rc == 2) return nsa::set_error(NSA_ERR_HIP, hipGetErrorString(hipGetLastError()));
  return NSA_OK;
}
