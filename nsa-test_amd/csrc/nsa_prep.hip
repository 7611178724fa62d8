// Layout preparation kernels: re-pack the per-group K/V operands into the compact,
// zero-padded layouts the attention kernels stage from, and the per-row backward
// statistics.  All of these are HBM streams over group-sized (not head-sized)
// tensors, except bwd_rowstats which reads O and dO once.
#include <type_traits>

#include "nsa_attn.h"
#include "nsa_device.h"
#include "nsa_kernels.h"

namespace nsa {

// Source matrix per (b,g): element (r, c) at src + b*s_b + g*s_g + r*s_r + c*s_c,
// r < R (time), c < C (feature).  Writes, for r < Rp (rows >= R zero-filled):
//   rowm[bg][r][c]  (if non-null)     colm[bg][c][r]  (if non-null)
//   rowf (if non-null): the rowfrag layout, colf (if non-null): the colfrag layout.
template <typename S>
__global__ __launch_bounds__(256) void repack_kernel(const S* __restrict__ src, int64_t s_b, int64_t s_g,
                                                     int64_t s_r, int64_t s_c, int G, int R, int C, int Rp,
                                                     S* __restrict__ rowm, S* __restrict__ colm,
                                                     S* __restrict__ rowf, S* __restrict__ colf) {
  using T = typename std::conditional<sizeof(S) == 2, bf16, float>::type;
  __shared__ S tile[64][65];
  const int bg = blockIdx.z;
  const int b = bg / G, g = bg % G;
  const int r0 = blockIdx.x * 64, c0 = blockIdx.y * 64;
  const S* base = src + b * s_b + g * s_g;
  const int tid = threadIdx.x;
  // read: walk along whichever source axis is contiguous
  const bool r_fast = s_r == 1;
  for (int i = tid; i < 64 * 64; i += 256) {
    const int rr = r_fast ? (i & 63) : (i >> 6);
    const int cc = r_fast ? (i >> 6) : (i & 63);
    const int r = r0 + rr, c = c0 + cc;
    S v;
    if (r < R && c < C) {
      v = base[r * s_r + c * s_c];
    } else {
      v = S(0);
    }
    tile[rr][cc] = v;
  }
  __syncthreads();
  const int64_t obase = (int64_t)bg * Rp * C;
  if (rowm) {
    for (int i = tid; i < 64 * 64; i += 256) {
      const int rr = i >> 6, cc = i & 63;
      const int r = r0 + rr, c = c0 + cc;
      if (r < Rp && c < C) rowm[obase + (int64_t)r * C + c] = tile[rr][cc];
    }
  }
  if (colm) {
    // key-major operands are stored C-permuted within each 32-key chunk (bf16)
    for (int i = tid; i < 64 * 64; i += 256) {
      const int cc = i >> 6, rr = i & 63;
      const int r = r0 + rr, c = c0 + cc;
      const int rpos = sizeof(S) == 2 ? ((r & ~31) | cperm_pos32(r & 31)) : r;
      if (r < Rp && c < C) colm[obase + (int64_t)c * Rp + rpos] = tile[rr][cc];
    }
  }
  // fragment-native layouts: consecutive threads write consecutive elements
  if (rowf) {
    for (int i = tid; i < 64 * 64; i += 256) {
      const int rr = i >> 6, cc = i & 63;
      const int r = r0 + rr, c = c0 + cc;
      if (r < Rp && c < C) rowf[obase + rowfrag_off<T>(r, c, C)] = tile[rr][cc];
    }
  }
  if (colf) {
    for (int i = tid; i < 64 * 64; i += 256) {
      const int cc = i >> 6, rr = i & 63;
      const int r = r0 + rr, c = c0 + cc;
      if (r < Rp && c < C) colf[obase + colfrag_off<T>(r, c, C)] = tile[rr][cc];
    }
  }
}

void launch_repack(int dtype, const void* src, int64_t s_b, int64_t s_g, int64_t s_r, int64_t s_c, int B, int G,
                   int R, int C, int Rp, void* rowm, void* colm, void* rowf, void* colf, hipStream_t st) {
  if (!rowm && !colm && !rowf && !colf) return;
  dim3 grid((Rp + 63) / 64, (C + 63) / 64, B * G);
  if (dtype == kF32) {
    hipLaunchKernelGGL(repack_kernel<float>, grid, dim3(256), 0, st, (const float*)src, s_b, s_g, s_r, s_c, G, R, C,
                       Rp, (float*)rowm, (float*)colm, (float*)rowf, (float*)colf);
  } else {
    hipLaunchKernelGGL(repack_kernel<uint16_t>, grid, dim3(256), 0, st, (const uint16_t*)src, s_b, s_g, s_r, s_c, G,
                       R, C, Rp, (uint16_t*)rowm, (uint16_t*)colm, (uint16_t*)rowf, (uint16_t*)colf);
  }
}

// Backward row statistics: delta = sum_d O*dO (fp32) and lse2 = (M+L)*log2(e)
// (+inf when L = -inf, i.e. the row saw no key: every probability is then 0).
template <typename T>
__global__ __launch_bounds__(256) void bwd_rowstats_kernel(AttnArgs a, int DV, int lpr_log2) {
  // LPR = 2^lpr_log2 lanes share one row, each reading 16-byte pieces; 256 / LPR rows
  // per workgroup
  using S = typename Store<T>::type;
  constexpr int EPF = 16 / sizeof(S);
  const int lpr = 1 << lpr_log2;
  const int sub = threadIdx.x & (lpr - 1);
  const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> lpr_log2;  // flattened (b, h, t)
  const int64_t nrows = (int64_t)a.B * a.H * a.Tq;
  const bool valid = row < nrows;
  const int64_t rr = valid ? row : nrows - 1;
  const int t = rr % a.Tq;
  const int h = (rr / a.Tq) % a.H;
  const int b = rr / ((int64_t)a.Tq * a.H);
  const S* o = reinterpret_cast<const S*>(a.o) + b * a.so_b + h * a.so_h + (int64_t)t * a.so_t;
  const S* d = reinterpret_cast<const S*>(a.dout) + b * a.sdo_b + h * a.sdo_h + (int64_t)t * a.sdo_t;
  float acc = 0.f;
  for (int e = sub * EPF; e < DV; e += lpr * EPF) {
    const uint4 ov = *reinterpret_cast<const uint4*>(o + e);
    const uint4 dv = *reinterpret_cast<const uint4*>(d + e);
    const S* op = reinterpret_cast<const S*>(&ov);
    const S* dp = reinterpret_cast<const S*>(&dv);
#pragma unroll
    for (int u = 0; u < EPF; ++u) acc += Elem<T>::to_f32(op[u]) * Elem<T>::to_f32(dp[u]);
  }
  for (int off = lpr >> 1; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
  if (valid && sub == 0) {
    float* delta = const_cast<float*>(a.delta);
    float* lse2 = const_cast<float*>(a.lse2);
    delta[row] = acc;
    const float L = a.L[b * a.sl_b + h * a.sl_h + (int64_t)t * a.sl_t];
    const float M = a.M[b * a.sm_b + h * a.sm_h + (int64_t)t * a.sm_t];
    lse2[row] = (L == -INFINITY) ? INFINITY : (M + L) * kLog2e;
  }
}

void launch_bwd_rowstats(int dtype, const AttnArgs& a, int DV, hipStream_t st) {
  const int64_t nrows = (int64_t)a.B * a.H * a.Tq;
  const int pieces = DV / (dtype == kF32 ? 4 : 8);  // DV is a multiple of 32 (padded head dims)
  int lg = 0;
  while ((1 << lg) < pieces && lg < 6) ++lg;
  const int64_t rows_per_wg = 256 >> lg;
  dim3 grid((unsigned)((nrows + rows_per_wg - 1) / rows_per_wg));
  if (dtype == kF32)
    hipLaunchKernelGGL(bwd_rowstats_kernel<float>, grid, dim3(256), 0, st, a, DV, lg);
  else
    hipLaunchKernelGGL(bwd_rowstats_kernel<bf16>, grid, dim3(256), 0, st, a, DV, lg);
}

}  // namespace nsa
