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

constexpr int kMaxRows = 64;  // R = TT * hpg accumulators per thread

template <typename S>
__device__ __forceinline__ float ldf(const S* p, int64_t off);
template <> __device__ __forceinline__ float ldf<float>(const float* p, int64_t off) { return p[off]; }
template <> __device__ __forceinline__ float ldf<uint16_t>(const uint16_t* p, int64_t off) {
  return bf16_bits_to_f32(p[off]);
}

template <typename S, int R>
__global__ __launch_bounds__(256) void score_topn_kernel(ScoreArgs a) {
  extern __shared__ float lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int bg = blockIdx.y, b = bg / a.G, g = bg % a.G;
  const int t0 = blockIdx.x * a.TT;
  const int TT = min(a.TT, a.T - t0);
  const int rows = TT * a.hpg;  // r = tt * hpg + hh
  const int t_last = t0 + TT - 1;
  const int NB = a.NB, nsel = a.nsel, dk = a.dk;
  // columns with any visible row (plus block 0 for the no-visible-block rule)
  __shared__ int s_ncomp;
  if (tid == 0) s_ncomp = 0;
  __syncthreads();
  {
    int mx = 0;
    for (int i = tid; i < NB; i += 256)
      if (a.block_ends[i] <= t_last) mx = i + 1;
    if (mx) atomicMax(&s_ncomp, mx);
  }
  __syncthreads();
  int ncomp = s_ncomp;
  if (ncomp == 0 && NB > 0) ncomp = 1;

  float* qs = lds;                           // [R][dk]
  float* ev = qs + rows * dk;                // [rows][ncomp]
  float* agg = ev + (int64_t)rows * ncomp;   // [TT][nsel]
  int* top = reinterpret_cast<int*>(agg + a.TT * nsel);  // [TT][64]

  const S* q = reinterpret_cast<const S*>(a.q);
  for (int x = tid; x < rows * dk; x += 256) {
    const int r = x / dk, e = x % dk;
    const int t = t0 + r / a.hpg, h = g * a.hpg + r % a.hpg;
    qs[r * dk + e] = ldf<S>(q, b * a.sq_b + (int64_t)h * a.sq_h + (int64_t)t * a.sq_t + (int64_t)e * a.sq_d);
  }
  __syncthreads();

  // ---- Eq. 8 logits: a thread owns one compressed block and a group of rows ----
  // (rows are split over threads when there are fewer than 256 columns, so the
  // early, short rows of a causal sequence still occupy the whole workgroup).
  // The key row is read as 16-byte vectors (the feature axis has unit stride); each
  // logit is still one sequential fma chain over e = 0..dk-1.
  {
    constexpr int EV = 16 / sizeof(S);
    const S* kc = reinterpret_cast<const S*>(a.kc) + b * a.sk_b + g * a.sk_g;
    int nrg = 1;
    while (nrg < R && nrg * 2 * ncomp <= 256 && (rows % (nrg * 2)) == 0) nrg *= 2;
    const int cpt = 256 / nrg;           // columns per pass
    const int rg = tid / cpt;
    const int nr = rows / nrg;           // rows per thread
    const int r0 = rg * nr;
    for (int i = tid % cpt; i < ncomp; i += cpt) {
      float acc[R];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = 0.0f;
      const S* krow = kc + (int64_t)i * a.sk_i;
      for (int e0 = 0; e0 < dk; e0 += EV) {
        const uint4 raw = *reinterpret_cast<const uint4*>(krow + e0);
        float kv[EV];
        if (sizeof(S) == 2) {
          const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            kv[2 * u] = __uint_as_float(w[u] << 16);
            kv[2 * u + 1] = __uint_as_float(w[u] & 0xffff0000u);
          }
        } else {
          kv[0] = __uint_as_float(raw.x);
          kv[1] = __uint_as_float(raw.y);
          kv[2] = __uint_as_float(raw.z);
          kv[3] = __uint_as_float(raw.w);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (r < nr) {
            const float* qr = qs + (r0 + r) * dk + e0;
#pragma unroll
            for (int u = 0; u < EV; ++u) acc[r] = fmaf(qr[u], kv[u], acc[r]);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (r < nr) ev[(r0 + r) * ncomp + i] = acc[r] * a.scale;
    }
  }
  __syncthreads();

  // ---- softmax per row (one wave per row) ----
  for (int r = wave; r < rows; r += 4) {
    const int t = t0 + r / a.hpg;
    const int h = g * a.hpg + r % a.hpg;
    float* row = ev + (int64_t)r * ncomp;
    bool anyv = false;
    float mx = -INFINITY;
    for (int i = lane; i < ncomp; i += 64) {
      const bool v = a.block_ends[i] <= t;
      anyv |= v;
      if (v) mx = fmaxf(mx, row[i]);
    }
    const bool any_row = __ballot(anyv) != 0ull;
    if (!any_row) mx = row[0];  // block 0 made visible
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    float part = 0.0f;
    for (int i = lane; i < ncomp; i += 64) {
      const bool v = a.block_ends[i] <= t || (!any_row && i == 0);
      const float e = v ? exp32(row[i] - mx) : 0.0f;
      row[i] = e;
      part += e;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) part = part + __shfl_xor(part, off);
    const float sum = part;
    for (int i = lane; i < ncomp; i += 64) row[i] = row[i] / sum;
    if (a.p_cmp) {
      float* pc = a.p_cmp + (((int64_t)b * a.H + h) * a.T + t) * NB;
      for (int i = lane; i < NB; i += 64) pc[i] = i < ncomp ? row[i] : 0.0f;
    }
  }
  __syncthreads();

  // ---- Eq. 9 per head, Eq. 10 over the group's heads ----
  for (int x = tid; x < TT * nsel; x += 256) {
    const int tt = x / nsel, j = x % nsel;
    const int t = t0 + tt;
    float ag = 0.0f;
    for (int hh = 0; hh < a.hpg; ++hh) {
      const float* row = ev + (int64_t)(tt * a.hpg + hh) * ncomp;
      float acc = 0.0f;
      for (int m = 0; m < a.s; ++m)
        for (int nn = 0; nn < a.a; ++nn) {
          const int ci = a.s * j + m + nn;
          if (ci < NB) acc += ci < ncomp ? row[ci] : 0.0f;
        }
      if (a.p_slc) a.p_slc[(((int64_t)b * a.H + g * a.hpg + hh) * a.T + t) * nsel + j] = acc;
      ag += acc;
    }
    agg[tt * nsel + j] = ag;
  }
  __syncthreads();

  // ---- top-n (one wave per timestep) ----
  const int kk = min(a.n, nsel);
  for (int tt = wave; tt < TT; tt += 4) {
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
      int64_t sel[64];
      int no = 0;
      int64_t cand[3];
      int nc = 0;
      if (a.include_fixed) {
        cand[nc++] = 0;
        cand[nc++] = t >= a.lprime ? (t - a.lprime) / a.lprime : 0;
        cand[nc++] = t / a.lprime;
      }
      for (int c = 0; c < nc + kk && no < a.n; ++c) {
        const int64_t v = c < nc ? cand[c] : (int64_t)top[tt * 64 + c - nc];
        bool dup = false;
        for (int u = 0; u < no; ++u) dup |= sel[u] == v;
        if (!dup) sel[no++] = v;
      }
      for (int u = 0; u < a.n; ++u) o[(int64_t)u * a.so_n] = u < no ? sel[u] : -1;
    }
  }
}

template <typename S, int R>
static hipError_t launch_score_R(const ScoreArgs& a, size_t lds, hipStream_t st) {
  auto fn = score_topn_kernel<S, R>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)lds);
  if (e != hipSuccess) return e;
  dim3 grid((a.T + a.TT - 1) / a.TT, a.B * a.G);
  hipLaunchKernelGGL(fn, grid, dim3(256), lds, st, a);
  return hipGetLastError();
}

template <typename S>
static hipError_t launch_score_T(const ScoreArgs& a, int rows, size_t lds, hipStream_t st) {
  if (rows <= 4) return launch_score_R<S, 4>(a, lds, st);
  if (rows <= 8) return launch_score_R<S, 8>(a, lds, st);
  if (rows <= 16) return launch_score_R<S, 16>(a, lds, st);
  if (rows <= 32) return launch_score_R<S, 32>(a, lds, st);
  return launch_score_R<S, 64>(a, lds, st);
}

// Returns 0 on success, 1 when the shape needs more LDS than a workgroup has,
// 2 on a HIP launch error.
int launch_score_topn(int dtype, ScoreArgs a, hipStream_t st) {
  constexpr size_t kLdsMax = 160 * 1024;
  int TT = a.hpg >= 16 ? 1 : 16 / a.hpg;
  for (;;) {
    const int rows = TT * a.hpg;
    const size_t lds = 4 * ((size_t)rows * a.dk + (size_t)rows * a.NB + (size_t)TT * a.nsel + (size_t)TT * 64);
    if (rows <= kMaxRows && lds <= kLdsMax) {
      a.TT = TT;
      hipError_t e = dtype == kF32 ? launch_score_T<float>(a, rows, lds, st) : launch_score_T<uint16_t>(a, rows, lds, st);
      return e == hipSuccess ? 0 : 2;
    }
    if (TT == 1) return 1;
    TT /= 2;
  }
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
  if (rc == 1) return nsa::set_error(NSA_ERR_UNSUPPORTED, "scores of one timestep exceed the LDS of a workgroup");
  if (rc == 2) return nsa::set_error(NSA_ERR_HIP, hipGetErrorString(hipGetLastError()));
  return NSA_OK;
}
