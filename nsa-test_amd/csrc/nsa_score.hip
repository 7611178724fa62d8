// Fused selection scoring on gfx950: Eq. 8 (compressed-attention probabilities),
// Eq. 9 (triangular remap to selection blocks), Eq. 10 (GQA head sum) and the top-n
// with fixed blocks, in two kernels after a small pre-kernel (score_tile_ncomp_kernel,
// the visible block count of each logits row tile):
//   score_logits_kernel  the Eq. 8 logits of every (row, visible compressed block) as an
//                        fp32 MFMA GEMM into the caller's workspace;
//   score_rows_kernel    softmax, Eq. 9, Eq. 10 and the top-n, one wave per
//                        (batch, group, timestep).
// Besides the workspace only the n indices per (b, g, t) are written (and, when the
// caller asks for them, the p_cmp / p_slc score tensors the reference module returns
// in attn_info).
//
// The fp32 arithmetic follows a fixed order so that the indices are reproducible
// bit for bit (this unit is compiled with -ffp-contract=off):
//   logit   acc = fma(q[e], k[e][i], acc) for e = 0..dk-1, then acc * scale
//   softmax e_i = exp32(s_i - max); sum = 64 lane partials (lane L adds the blocks
//           256 s + 4 L + u, s ascending then u = 0..3) combined by xor-butterfly
//           over 32,16,8,4,2,1;
//           p = e * (1 / sum), the reciprocal correctly rounded
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

// exp32 of a softmax argument x = s - max <= 0 (or -inf): k = rint(x log2 e), r by a
// two-constant Cody-Waite reduction, the polynomial by fma, p * 2^k; 0 below -64.  Only
// arguments <= 0 occur, so there is no input clamp (an input below -64, -inf included,
// may give a non-finite intermediate that the final select replaces by 0), and p * 2^k
// is one ldexp (k >= -93 and p in [0.7, 1.5] keep it normal: exact, as the multiply by
// the constructed power of two the oracle performs).
__device__ __forceinline__ float exp32(float x) {
  const float kL2e = 1.44269504088896341f;
  const float kLn2Hi = 0.693145751953125f;
  const float kLn2Lo = 1.42860682030941723212e-6f;
  const bool ok = x >= -64.0f;
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
  const float v = __builtin_amdgcn_ldexpf(p, (int)k);
  return ok ? v : 0.0f;
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
  float* lg;     // workspace: scaled logits [B*G][T*hpg][ncs], row r = t * hpg + head in group
  int* tile_nc;  // workspace: per kLgTM-row tile, the compressed blocks [0, n) it must compute
  int B, H, G, hpg, T, dk, NB;
  float scale;
  int a, s, nsel, lprime, n, include_fixed;
  int ncs;  // logit row stride: NB rounded up to 64
  int q0;   // absolute position of query row 0 (positions decide visibility and fixed blocks)
};

constexpr int kMaxRows = 64;    // heads per group
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

// number of compressed blocks [0, ncomp) that hold every block visible at t_last
// (at least block 0, which the no-visible-block rule scores); s_out is LDS
__device__ __forceinline__ int score_ncomp(const ScoreArgs& a, int t_last, int* s_out) {
  if (threadIdx.x == 0) *s_out = 0;
  __syncthreads();
  int mx = 0;
  for (int i = threadIdx.x; i < a.NB; i += blockDim.x)
    if (a.block_ends[i] <= t_last) mx = i + 1;
  if (mx) atomicMax(s_out, mx);
  __syncthreads();
  const int nc = *s_out;
  return nc == 0 && a.NB > 0 ? 1 : nc;
}

// ---------------------------------------------------------------- logits ----
// Eq. 8 logits of one group as an fp32 GEMM on the matrix cores:
// lg[r][i] = scale * (sum over e = 0..dk-1 of q[r][e] k[i][e]), each element one
// sequential fma chain in e order (the accumulation order the indices are defined by).
// v_mfma_f32_16x16x4_f32 computes D = C + sum_k A[m][k] B[k][n] as four IEEE fp32
// fmas in k order 0..3, each rounded (subnormals kept; measured on gfx950 against an
// emulated fma chain over millions of random operands), so the chain of MFMAs over the
// feature steps e = 4j..4j+3 (slot k = e - 4j) is exactly that fma chain.
// Workgroup = 128 query rows x 64 compressed blocks, 4 waves of 32 rows x 64 blocks
// (4 x 2 MFMA tiles, blocks as the M operand so a lane holds 4 consecutive blocks of
// one row); the operands are staged through LDS as fp32 in EK-feature chunks (the next
// chunk is loaded into registers while the current one is used).  Column tiles past
// the last block visible to the tile's last timestep exit at once (the causal
// triangle is never computed).
constexpr int kLgTM = 128, kLgTN = 64, kLgEK = 32;

// Per kLgTM-row tile of the logits (rows r = t * hpg + head, the same for every batch
// and group): the number of compressed blocks holding every block visible to the tile's
// last timestep, computed once here instead of by each of the tile's column workgroups.
__global__ __launch_bounds__(256) void score_tile_ncomp_kernel(ScoreArgs a) {
  __shared__ int s_nc;
  const int row0 = blockIdx.x * kLgTM;
  const int t_last = min(a.T - 1, (row0 + kLgTM - 1) / a.hpg) + a.q0;
  const int nc = score_ncomp(a, t_last, &s_nc);
  if (threadIdx.x == 0) a.tile_nc[blockIdx.x] = nc;
}

template <typename S>
__global__ __launch_bounds__(256) void score_logits_kernel(ScoreArgs a) {
  constexpr int EPL = 16 / sizeof(S);           // elements per 16-byte piece
  constexpr int TPR = 256 / kLgTM;              // threads staging one A row
  constexpr int APT = kLgEK / EPL / TPR;        // A pieces per thread (part of its row's chunk)
  constexpr int BPT = kLgTN * (kLgEK / EPL) / 256;  // B pieces per thread
  constexpr int AP = kLgTM + 16, BP = kLgTN + 16;  // padded LDS rows: the 4 k slots of a read hit distinct banks
  __shared__ __attribute__((aligned(16))) float As[kLgEK * AP];  // [e][row]
  __shared__ __attribute__((aligned(16))) float Bs[kLgEK * BP];  // [e][col]

  const int tid = threadIdx.x;
  const int bg = blockIdx.z, b = bg / a.G, g = bg % a.G;
  const int hpg = a.hpg;
  const int Rall = a.T * hpg;
  const int row0 = blockIdx.x * kLgTM, col0 = blockIdx.y * kLgTN;
  if (col0 >= a.tile_nc[blockIdx.x]) return;  // workgroup-uniform: past the visible frontier

  // the thread's staging row (A) and column (B)
  const int arow = min(row0 + tid % kLgTM, Rall - 1), apart = tid / kLgTM;
  const S* qrow = reinterpret_cast<const S*>(a.q) + b * a.sq_b + (int64_t)(g * hpg + arow % hpg) * a.sq_h +
                  (int64_t)(arow / hpg) * a.sq_t;
  const int bcol = tid % kLgTN, bpart0 = tid / kLgTN;
  const S* kcol = reinterpret_cast<const S*>(a.kc) + b * a.sk_b + g * a.sk_g +
                  (int64_t)min(col0 + bcol, a.NB - 1) * a.sk_i;
  const int dk = a.dk;
  uint4 pa[APT], pb[BPT];
  auto load = [&](int e0) {
#pragma unroll
    for (int j = 0; j < APT; ++j)
      pa[j] = e0 + (apart + j * TPR) * EPL < dk ? *reinterpret_cast<const uint4*>(qrow + e0 + (apart + j * TPR) * EPL)
                                               : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      const int e = e0 + (bpart0 + j * (256 / kLgTN)) * EPL;
      pb[j] = e < dk ? *reinterpret_cast<const uint4*>(kcol + e) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int j = 0; j < APT; ++j) {
      float v[EPL];
      unpack16<S>(pa[j], v);
#pragma unroll
      for (int u = 0; u < EPL; ++u) As[((apart + j * TPR) * EPL + u) * AP + tid % kLgTM] = v[u];
    }
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      float v[EPL];
      unpack16<S>(pb[j], v);
#pragma unroll
      for (int u = 0; u < EPL; ++u) Bs[((bpart0 + j * (256 / kLgTN)) * EPL + u) * BP + bcol] = v[u];
    }
  };

  const int lane = tid & 63, li = lane & 15, kk = lane >> 4;
  constexpr int NT = kLgTM / 64;    // 16-row MFMA tiles per wave
  const int wr0 = (tid >> 6) * (kLgTM / 4);  // the wave's first row in the tile
  f32x4 acc[4][NT];                 // [block tile mt][row tile nt]
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[m][n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // a chunk past dk holds zeros: fma(0, 0, acc) == acc (acc is never -0), so the
  // padded steps leave every chain exactly as the dk-step one
  load(0);
  for (int e0 = 0; e0 < dk; e0 += kLgEK) {
    __syncthreads();  // the previous chunk's products are done
    store();
    __syncthreads();
    if (e0 + kLgEK < dk) load(e0 + kLgEK);
#pragma unroll
    for (int j4 = 0; j4 < kLgEK; j4 += 4) {
      const int e = j4 + kk;  // this lane's k slot
      float kv[4], qv[NT];
#pragma unroll
      for (int m = 0; m < 4; ++m) kv[m] = Bs[e * BP + m * 16 + li];
#pragma unroll
      for (int n = 0; n < NT; ++n) qv[n] = As[e * AP + wr0 + n * 16 + li];
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[m], qv[n], acc[m][n], 0, 0, 0);
    }
  }

  // acc[m][n][u]: block col0 + 16 m + 4 kk + u of row row0 + wr0 + 16 n + li
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int r = row0 + wr0 + n * 16 + li;
    if (r < Rall) {
      float* o = a.lg + ((int64_t)bg * Rall + r) * a.ncs + col0 + kk * 4;
#pragma unroll
      for (int m = 0; m < 4; ++m)
        *reinterpret_cast<float4*>(o + m * 16) =
            make_float4(acc[m][n][0] * a.scale, acc[m][n][1] * a.scale, acc[m][n][2] * a.scale,
                        acc[m][n][3] * a.scale);
    }
  }
}

// ------------------------------------------------------------------ rows ----
// One wave per (batch, group, timestep): a workgroup of NW waves takes NW consecutive
// timesteps, and after the block ends are staged in LDS no wave waits for another.  A
// wave walks its timestep's hpg rows in head order, each row in registers -- lane L
// holds the blocks 256 s + 4 L + u (s < NQ, u < 4), one 16-byte piece per s (a
// coalesced 1 KB load per wave), the next row's pieces loaded while the current one
// is processed:
//   1. invisible blocks set to -inf (logits are finite; exp32 maps -inf to 0), max;
//   2. e = exp32(s - max), lane partials over s then u, xor butterfly;
//   3. p = e * (1 / sum);
//   4. Eq. 9: for the (a, s) = (2, 4) remap output j = 64 s + L reads blocks 4j..4j+4,
//      the lane's own piece s plus the first block of the next lane's piece; other
//      remaps go through a wave-private LDS copy of the row;
//   5. Eq. 10: the row's Eq. 9 scores added to the timestep's running sums (heads in
//      order), in registers for the (2, 4) remap (output j of lane j % 64), in a
//      wave-private LDS row otherwise.
// Then the top-n of the timestep from those sums.  Blocks past the last one visible
// at t are not read (the logits kernel computed every visible block, and block 0).
constexpr int kRowsWaves = 8;

template <int NQ, bool FAST9>
__global__ __launch_bounds__(64 * kRowsWaves) __attribute__((amdgpu_waves_per_eu(NQ == 8 ? 4 : 1))) void score_rows_kernel(ScoreArgs a) {
  // LDS: sbe [NQ * 256] block ends (INT_MAX past NB); generic remap only, per wave:
  // row copy [NQ * 256] + Eq. 10 sums [nsel rounded up to 4]
  extern __shared__ float lds[];
  constexpr bool kPrefetch = NQ <= 8;  // registers for the next row's pieces
  const int tid = threadIdx.x, lane = tid & 63;
  const int NW = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bg = blockIdx.y, b = bg / a.G, g = bg % a.G;
  const int NB = a.NB, nsel = a.nsel, ncs = a.ncs, hpg = a.hpg;
  int* sbe = reinterpret_cast<int*>(lds);
  for (int i = tid; i < NQ * 256; i += blockDim.x) sbe[i] = i < NB ? a.block_ends[i] : 0x7fffffff;
  __syncthreads();
  const int t = blockIdx.x * NW + wave;  // row; its position is ta
  if (t >= a.T) return;  // whole wave; no barrier follows
  const int ta = t + a.q0;
  const int nsel4 = (nsel + 3) & ~3;
  float* wb = lds + NQ * 256 + wave * (NQ * 256 + nsel4);  // generic remap only
  float* wag = wb + NQ * 256;

  int vis_hi = 0;  // 1 + the largest block index visible at t (0: none)
  int nfull = NQ;  // leading pieces whose 256 blocks are all visible (no mask needed)
#pragma unroll
  for (int s = 0; s < NQ; ++s) {
    const int4 be = *reinterpret_cast<const int4*>(sbe + 256 * s + 4 * lane);
    const int i = 256 * s + 4 * lane;
    if (be.x <= ta) vis_hi = i + 1;
    if (be.y <= ta) vis_hi = i + 2;
    if (be.z <= ta) vis_hi = i + 3;
    if (be.w <= ta) vis_hi = i + 4;
    const bool all4 = be.x <= ta && be.y <= ta && be.z <= ta && be.w <= ta;
    if (nfull == NQ && __ballot(!all4)) nfull = s;  // wave-uniform
  }
  vis_hi = wave_butterfly(vis_hi, [](int x, int y) { return max(x, y); });
  vis_hi = __builtin_amdgcn_readfirstlane(vis_hi);  // uniform: branches on it stay scalar
  // columns read (block 0 always: the no-visible-block rule scores it)
  const int ncol = max(64, ((vis_hi + 63) >> 6) * 64);
  // pieces holding a read column; the others hold only invisible blocks, whose p is an
  // exact 0 that adds nothing to the sum, Eq. 9 or Eq. 10 (wave-uniform skip)
  const int nact = (ncol + 255) >> 8;
  const float* lgb = a.lg + ((int64_t)bg * a.T + t) * hpg * ncs;

  float agg[FAST9 ? NQ : 1];
#pragma unroll
  for (int s = 0; s < (FAST9 ? NQ : 1); ++s) agg[s] = 0.0f;
  if constexpr (!FAST9)
    for (int j = lane; j < nsel; j += 64) wag[j] = 0.0f;
  float4 cur[NQ], nxt[kPrefetch ? NQ : 1];
  // one 16-byte load per active piece; columns past ncol (not computed for this row,
  // or past the row when ncs is not a multiple of 256) are read from a clamped address
  // and are masked below (their blocks are invisible at t)
  auto load_row = [&](float4* v, int hh) __attribute__((always_inline)) {
    const float* row = lgb + (int64_t)hh * ncs;
#pragma unroll
    for (int s = 0; s < NQ; ++s)
      if (s < nact) v[s] = *reinterpret_cast<const float4*>(row + min(256 * s + 4 * lane, ncs - 4));
  };
  load_row(cur, 0);
  for (int hh = 0; hh < hpg; ++hh) {
    if constexpr (kPrefetch)
      if (hh + 1 < hpg) load_row(nxt, hh + 1);
    const int h = g * hpg + hh;
    float v[NQ][4];
    float mx = -INFINITY;
#pragma unroll
    for (int s = 0; s < NQ; ++s) {
      if (s >= nact) {
        v[s][0] = v[s][1] = v[s][2] = v[s][3] = 0.0f;
        continue;
      }
      if (s < nfull) {  // every block of the piece visible
        v[s][0] = cur[s].x;
        v[s][1] = cur[s].y;
        v[s][2] = cur[s].z;
        v[s][3] = cur[s].w;
      } else {
        const int4 be = *reinterpret_cast<const int4*>(sbe + 256 * s + 4 * lane);
        v[s][0] = be.x <= ta ? cur[s].x : -INFINITY;
        v[s][1] = be.y <= ta ? cur[s].y : -INFINITY;
        v[s][2] = be.z <= ta ? cur[s].z : -INFINITY;
        v[s][3] = be.w <= ta ? cur[s].w : -INFINITY;
      }
      mx = fmaxf(mx, fmaxf(fmaxf(v[s][0], v[s][1]), fmaxf(v[s][2], v[s][3])));
    }
    if (vis_hi == 0) {  // no visible block (wave-uniform): block 0 is scored
      mx = __shfl(cur[0].x, 0);
      if (lane == 0) v[0][0] = mx;
    }
    mx = wave_butterfly(mx, [](float x, float y) { return fmaxf(x, y); });
    float part = 0.0f;
#pragma unroll
    for (int s = 0; s < NQ; ++s)
      if (s < nact)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          v[s][u] = exp32(v[s][u] - mx);
          part += v[s][u];
        }
    part = wave_butterfly(part, [](float x, float y) { return x + y; });
    const float rs = 1.0f / part;
#pragma unroll
    for (int s = 0; s < NQ; ++s)
      if (s < nact)
#pragma unroll
        for (int u = 0; u < 4; ++u) v[s][u] *= rs;  // invisible blocks: p = 0 exactly
    if (a.p_cmp) {
      float* pc = a.p_cmp + (((int64_t)b * a.H + h) * a.T + t) * NB;
#pragma unroll
      for (int s = 0; s < NQ; ++s)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int i = 256 * s + 4 * lane + u;
          if (i < NB) pc[i] = v[s][u];
        }
    }
    // Eq. 9 in the reference's (m, n) order, starting from 0; invisible blocks (and
    // blocks past NB) add an exact +0
    float* psl = a.p_slc ? a.p_slc + (((int64_t)b * a.H + h) * a.T + t) * nsel : nullptr;
    if constexpr (FAST9) {  // (m, n) -> 4j + {0, 1, 1, 2, 2, 3, 3, 4}
#pragma unroll
      for (int s = 0; s < NQ; ++s) {
        if (s >= nact) {  // Eq. 9 scores of exact 0
          const int j = 64 * s + lane;
          if (psl && j < nsel) psl[j] = 0.0f;
          continue;
        }
        float nb = __shfl_down(v[s][0], 1);
        const float nb63 = s + 1 < NQ ? __shfl(v[s + 1 < NQ ? s + 1 : s][0], 0) : 0.0f;
        if (lane == 63) nb = nb63;
        const float s9 = (((((((0.0f + v[s][0]) + v[s][1]) + v[s][1]) + v[s][2]) + v[s][2]) + v[s][3]) + v[s][3]) + nb;
        agg[s] += s9;
        const int j = 64 * s + lane;
        if (psl && j < nsel) psl[j] = s9;
      }
    } else {
#pragma unroll
      for (int s = 0; s < NQ; ++s)
        *reinterpret_cast<float4*>(wb + 256 * s + 4 * lane) = make_float4(v[s][0], v[s][1], v[s][2], v[s][3]);
      wave_lds_sync();
      for (int j = lane; j < nsel; j += 64) {
        float s9 = 0.0f;
        for (int m = 0; m < a.s; ++m)
          for (int nn = 0; nn < a.a; ++nn) {
            const int ci = a.s * j + m + nn;
            if (ci < NB) s9 += wb[ci];
          }
        wag[j] += s9;
        if (psl) psl[j] = s9;
      }
      wave_lds_sync();  // the copy is rewritten for the next row
    }
    if constexpr (kPrefetch) {
#pragma unroll
      for (int s = 0; s < NQ; ++s) cur[s] = nxt[s];
    } else if (hh + 1 < hpg) {
      load_row(cur, hh + 1);
    }
  }

  // ---- top-n: the kk largest sums, equal sums lower index first ----
  const int kk = min(a.n, nsel);
  const int nc = a.include_fixed ? 3 : 0;
  if constexpr (FAST9) {
#pragma unroll
    for (int s = 0; s < NQ; ++s)
      if (64 * s + lane >= nsel) agg[s] = -INFINITY;  // past nsel: never taken (kk <= nsel)
  }
  int top0 = -1, top1 = -1;  // lane c holds candidate c (top0) and c + 64 (top1)
  for (int rk = 0; rk < kk; ++rk) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    if constexpr (FAST9) {
#pragma unroll
      for (int s = 0; s < NQ; ++s) {
        const int j = 64 * s + lane;
        if (agg[s] > bv || (agg[s] == bv && j < bi)) {
          bv = agg[s];
          bi = j;
        }
      }
    } else {
      for (int j = lane; j < nsel; j += 64) {
        const float x = wag[j];
        if (x > bv || (x == bv && j < bi)) {
          bv = x;
          bi = j;
        }
      }
    }
    auto take = [&](float ov, int oi) __attribute__((always_inline)) {
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    };
    take(lane_xor<32>(bv), lane_xor<32>(bi));
    take(lane_xor<16>(bv), lane_xor<16>(bi));
    take(lane_xor<8>(bv), lane_xor<8>(bi));
    take(lane_xor<4>(bv), lane_xor<4>(bi));
    take(lane_xor<2>(bv), lane_xor<2>(bi));
    take(lane_xor<1>(bv), lane_xor<1>(bi));
    // bi is wave-uniform: its owner marks it taken
    if constexpr (FAST9) {
#pragma unroll
      for (int s = 0; s < NQ; ++s)
        if (64 * s + lane == bi) agg[s] = -INFINITY;
    } else {
      if (lane == (bi & 63)) wag[bi] = -INFINITY;
      wave_lds_sync();
    }
    const int c = nc + rk;
    if (lane == (c & 63)) {
      if (c < 64) top0 = bi;
      else top1 = bi;
    }
  }
  // candidates: fixed [0, max(0,(t-l')/l'), t/l'] then the top-k.  The top-k are
  // distinct, so a candidate can only repeat one of the fixed ones before it.
  const int f1 = ta >= a.lprime ? (ta - a.lprime) / a.lprime : 0;
  const int f2 = ta / a.lprime;
  const int ncand = nc + kk;  // <= 67 (n <= 64)
  int64_t* o = a.out + b * a.so_b + g * a.so_g + (int64_t)t * a.so_t;
  int kept = 0;  // candidates kept so far (wave-uniform)
  for (int c0 = 0; c0 < ncand && kept < a.n; c0 += 64) {
    const int c = c0 + lane;
    int v = -1;
    bool keep = false;
    if (c < ncand) {
      v = c < nc ? (c == 0 ? 0 : c == 1 ? f1 : f2) : (c0 == 0 ? top0 : top1);
      const bool dup = nc > 0 && ((c > 0 && v == 0) || (c > 1 && v == f1) || (c > 2 && v == f2));
      keep = !dup;
    }
    const uint64_t km = __ballot(keep);
    const int rank = kept + __builtin_popcountll(km & ((1ull << lane) - 1ull));
    if (keep && rank < a.n) o[(int64_t)rank * a.so_n] = v;
    kept += __builtin_popcountll(km);
  }
  for (int u = min(kept, a.n) + lane; u < a.n; u += 64) o[(int64_t)u * a.so_n] = -1;
}

static int score_ncs(int NB) { return NB > 0 ? ((NB + 63) / 64) * 64 : 64; }

static int score_rows_nq(int ncs) {  // 16-byte pieces per lane: a power of two >= ncs / 256
  int nq = 1;
  while (nq * 256 < ncs) nq *= 2;
  return nq;
}

// LDS of a rows workgroup of nw waves
static size_t score_rows_lds(int nq, bool fast9, int nw, int nsel) {
  const size_t per_wave = fast9 ? 0 : (size_t)nq * 256 + (size_t)((nsel + 3) & ~3);
  return 4 * ((size_t)nq * 256 + nw * per_wave);
}

template <int NQ, bool FAST9>
static hipError_t launch_rows_k(const ScoreArgs& a, int nw, size_t lds, hipStream_t st) {
  auto fn = score_rows_kernel<NQ, FAST9>;
  if (lds > 64 * 1024) {  // beyond the default dynamic LDS limit
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return e;
  }
  dim3 grid((a.T + nw - 1) / nw, a.B * a.G);
  hipLaunchKernelGGL(fn, grid, dim3(64 * nw), lds, st, a);
  return hipGetLastError();
}

template <bool FAST9>
static hipError_t launch_rows_q(const ScoreArgs& a, int nq, int nw, size_t lds, hipStream_t st) {
  switch (nq) {
    case 1: return launch_rows_k<1, FAST9>(a, nw, lds, st);
    case 2: return launch_rows_k<2, FAST9>(a, nw, lds, st);
    case 4: return launch_rows_k<4, FAST9>(a, nw, lds, st);
    case 8: return launch_rows_k<8, FAST9>(a, nw, lds, st);
    case 16: return launch_rows_k<16, FAST9>(a, nw, lds, st);
  }
  return hipErrorInvalidValue;
}

// Launches the logits GEMM and the rows kernel (one wave per timestep).
// Returns 0 on success, 1 when no configuration fits, 2 on a HIP launch error.
int launch_score_topn(int dtype, ScoreArgs a, hipStream_t st) {
  if (a.NB > kMaxCols || a.hpg > kMaxRows) return 1;
  a.ncs = score_ncs(a.NB);
  {
    const int Rall = a.T * a.hpg;
    const dim3 grid((Rall + kLgTM - 1) / kLgTM, a.ncs / kLgTN, a.B * a.G);
    hipLaunchKernelGGL(score_tile_ncomp_kernel, dim3(grid.x), dim3(256), 0, st, a);
    if (dtype == kF32) hipLaunchKernelGGL(score_logits_kernel<float>, grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(score_logits_kernel<uint16_t>, grid, dim3(256), 0, st, a);
    if (hipGetLastError() != hipSuccess) return 2;
  }
  const int nq = score_rows_nq(a.ncs);
  const bool fast9 = a.a == 2 && a.s == 4;
  // fewer waves per workgroup when the generic remap's LDS rows do not fit, and 4 when the
  // row registers allow at most 3 waves per SIMD (a workgroup of 4 puts one on each SIMD,
  // so three workgroups share a CU where one of 8 waves would leave a third slot empty)
  int nw = nq >= 8 ? 4 : kRowsWaves;
  while (nw > 1 && score_rows_lds(nq, fast9, nw, a.nsel) > 80 * 1024) nw /= 2;
  const size_t lds = score_rows_lds(nq, fast9, nw, a.nsel);
  if (lds > 156 * 1024) return 1;
  const hipError_t e = fast9 ? launch_rows_q<true>(a, nq, nw, lds, st) : launch_rows_q<false>(a, nq, nw, lds, st);
  return e == hipSuccess ? 0 : 2;
}

}  // namespace nsa

// ------------------------------------------------------------------ C ABI ----
#include "../../include/nsa_hip.h"

#include "nsa_kernels.h"

// the fp32 logits of every (row, compressed block): Z*H*T rows of NB rounded up to 64,
// then one int per kLgTM-row logits tile of a group
static size_t score_ws_logits(int Z, int H, int n_ctx, int n_blocks) {
  return (size_t)Z * H * n_ctx * nsa::score_ncs(n_blocks) * 4;
}
static size_t score_ws_bytes(int Z, int H, int G, int n_ctx, int n_blocks) {
  const size_t ntiles = ((size_t)n_ctx * (H / G) + nsa::kLgTM - 1) / nsa::kLgTM;
  return score_ws_logits(Z, H, n_ctx, n_blocks) + ((ntiles * 4 + 255) & ~(size_t)255);
}

extern "C" size_t nsa_score_topn_workspace_size(int Z, int H, int n_kv_groups, int n_ctx, int head_dim_qk,
                                                int n_blocks, int n) {
  (void)head_dim_qk;
  (void)n;
  if (Z <= 0 || H <= 0 || n_kv_groups <= 0 || H % n_kv_groups || n_ctx <= 0 || n_blocks < 0) return 0;
  return score_ws_bytes(Z, H, n_kv_groups, n_ctx, n_blocks);
}

static int score_topn_impl(const void* q, const void* k_cmp, const int32_t* block_ends, int64_t* out_idx,
                              float* p_cmp, float* p_slc, int64_t stride_qz, int64_t stride_qh, int64_t stride_qm,
                              int64_t stride_qk, int64_t stride_kz, int64_t stride_kg, int64_t stride_kk,
                              int64_t stride_kn, int64_t stride_iz, int64_t stride_ig, int64_t stride_im,
                              int64_t stride_in, int Z, int H, int n_kv_groups, int n_ctx, int head_dim_qk,
                              int n_blocks, int l, int d, int l_prime, int n, int include_fixed, int n_fixed,
                              int dtype, float scale,
                              int q_offset, void* workspace, size_t workspace_bytes, nsa_stream_t stream) {
  using namespace nsa;
  if (dtype != NSA_F32 && dtype != NSA_BF16) return nsa::set_error(NSA_ERR_INVALID, "dtype not supported");
  if (Z <= 0 || H <= 0 || n_kv_groups <= 0 || H % n_kv_groups || n_ctx < 0 || head_dim_qk <= 0 || n_blocks < 0)
    return nsa::set_error(NSA_ERR_INVALID, "bad shape");
  if (d <= 0 || l <= 0 || l_prime <= 0 || l % d || l_prime % d)
    return nsa::set_error(NSA_ERR_INVALID, "need l % d == 0 and l_prime % d == 0");
  if (q_offset < 0) return nsa::set_error(NSA_ERR_INVALID, "q_offset must be >= 0");
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
  {
    const size_t need = score_ws_bytes(Z, H, n_kv_groups, n_ctx, n_blocks);
    if (workspace_bytes < need || (need && (!workspace || ((uintptr_t)workspace) % 16))) {
      char msg[128];
      snprintf(msg, sizeof(msg), "workspace of %zu bytes (16-byte aligned) required, %zu given", need,
               workspace_bytes);
      return nsa::set_error(NSA_ERR_WORKSPACE, msg);
    }
  }
  ScoreArgs a{};
  a.lg = static_cast<float*>(workspace);
  a.tile_nc = reinterpret_cast<int*>(static_cast<char*>(workspace) + score_ws_logits(Z, H, n_ctx, n_blocks));
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
  a.q0 = q_offset;
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

extern "C" int nsa_score_topn(const void* q, const void* k_cmp, const int32_t* block_ends, int64_t* out_idx,
                              float* p_cmp, float* p_slc, int64_t stride_qz, int64_t stride_qh, int64_t stride_qm,
                              int64_t stride_qk, int64_t stride_kz, int64_t stride_kg, int64_t stride_kk,
                              int64_t stride_kn, int64_t stride_iz, int64_t stride_ig, int64_t stride_im,
                              int64_t stride_in, int Z, int H, int n_kv_groups, int n_ctx, int head_dim_qk,
                              int n_blocks, int l, int d, int l_prime, int n, int include_fixed, int n_fixed,
                              int dtype, float scale, void* workspace, size_t workspace_bytes, nsa_stream_t stream) {
  return score_topn_impl(q, k_cmp, block_ends, out_idx, p_cmp, p_slc, stride_qz, stride_qh, stride_qm, stride_qk,
                         stride_kz, stride_kg, stride_kk, stride_kn, stride_iz, stride_ig, stride_im, stride_in, Z,
                         H, n_kv_groups,
                         n_ctx, head_dim_qk, n_blocks, l, d, l_prime, n, include_fixed, n_fixed, dtype, scale, 0,
                         workspace,
                         workspace_bytes, stream);
}

extern "C" int nsa_score_topn_ex(const void* q, const void* k_cmp, const int32_t* block_ends, int64_t* out_idx,
                              float* p_cmp, float* p_slc, int64_t stride_qz, int64_t stride_qh, int64_t stride_qm,
                              int64_t stride_qk, int64_t stride_kz, int64_t stride_kg, int64_t stride_kk,
                              int64_t stride_kn, int64_t stride_iz, int64_t stride_ig, int64_t stride_im,
                              int64_t stride_in, int Z, int H, int n_kv_groups, int n_ctx, int head_dim_qk,
                              int n_blocks, int l, int d, int l_prime, int n, int include_fixed, int n_fixed,
                              int dtype, float scale,
                              int q_offset, void* workspace, size_t workspace_bytes, nsa_stream_t stream) {
  return score_topn_impl(q, k_cmp, block_ends, out_idx, p_cmp, p_slc, stride_qz, stride_qh, stride_qm, stride_qk,
                         stride_kz, stride_kg, stride_kk, stride_kn, stride_iz, stride_ig, stride_im, stride_in, Z,
                         H, n_kv_groups,
                         n_ctx, head_dim_qk, n_blocks, l, d, l_prime, n, include_fixed, n_fixed, dtype, scale,
                         q_offset, workspace,
                         workspace_bytes, stream);
}
