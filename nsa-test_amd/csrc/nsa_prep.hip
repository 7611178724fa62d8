// Layout preparation kernels: re-pack the per-group K/V operands into the compact,
// zero-padded layouts the attention kernels stage from.  All of these are HBM streams
// over group-sized (not head-sized) tensors.
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

}  // namespace nsa
