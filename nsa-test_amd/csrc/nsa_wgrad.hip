// Weight gradient of a token-wise linear layer, dW = dY^T X over every token row: the
// compression MLP's first layer reduces over all B*G*T tokens (32768 rows against a
// 384 x 192 weight at the paper configuration), a shape whose output has too few tiles
// for one GEMM to fill the GPU.  The rows are split into S chunks: workgroup (i, j, c)
// sums chunk c of the output tile (i, j) (64 rows by up to 192 columns) on the matrix
// cores (fp32), and a second pass adds the S partial tiles in chunk order
// (deterministic) and rounds once.
//
// Both operands are read row-major (token rows, features contiguous) into LDS; the MFMA
// fragments, whose K slots run along the token axis, come from LDS transpose loads.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/nsa_hip.h"
#include "nsa_device.h"
#include "nsa_kernels.h"

namespace nsa {

constexpr int kWgTile = 64;   // output rows per workgroup (dY features); n1, n2 multiples of it
constexpr int kWgRows = 64;   // token rows staged per step
constexpr int kWgPitchA = kWgTile + 8;  // LDS row pitches (elements): 16-byte aligned rows, spread banks

// the widest column block (192, 128 or 64 columns) that divides n2
static int wgrad_block_cols(int n2) { return n2 % 192 == 0 ? 192 : n2 % 128 == 0 ? 128 : 64; }

// rows per chunk, a multiple of the staging step: enough chunks for about 512 workgroups
// over the output tiles, at most 64 (each chunk writes a partial of the whole output)
static int wgrad_chunk_rows(int rows, int n1, int n2) {
  const int tiles = (n1 / kWgTile) * (n2 / wgrad_block_cols(n2));
  int s = (512 + tiles - 1) / tiles;
  s = s < 1 ? 1 : s > 64 ? 64 : s;
  const int per = (rows + s - 1) / s;
  return ((per + kWgRows - 1) / kWgRows) * kWgRows;
}

// Workgroup (i, j, c): output rows 64 i .. + 63 and columns 16 NS j .. + 16 NS - 1 over the
// token rows of chunk c; wave w owns output rows 64 i + 16 w .. + 15 and all NS column
// subtiles, so every staged X row is read from HBM once per 64 output rows.
template <int NS>
__global__ __launch_bounds__(256) void wgrad_partial_kernel(const uint16_t* __restrict__ dy, int64_t ld_dy,
                                                            const uint16_t* __restrict__ x, int64_t ld_x, int rows,
                                                            int n1, int n2, int chunk_rows,
                                                            float* __restrict__ part) {
  constexpr int WB = 16 * NS;    // output columns of the workgroup
  constexpr int PB = WB + 8;     // X tile pitch
  constexpr int PA = kWgPitchA;  // dY tile pitch
  constexpr int NPA = kWgRows * kWgTile / 8 / 256;  // 16-byte pieces per thread and step
  constexpr int NPB = kWgRows * WB / 8 / 256;
  __shared__ __attribute__((aligned(16))) uint16_t sa[2][kWgRows * PA];
  __shared__ __attribute__((aligned(16))) uint16_t sb[2][kWgRows * PB];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, j = lane & 15;
  const int c1 = blockIdx.x * kWgTile, c2 = blockIdx.y * WB;
  const int r_lo = blockIdx.z * chunk_rows, r_hi = min(rows, r_lo + chunk_rows);
  uint4 va[NPA], vb[NPB];
  auto load = [&](int r0) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < NPA; ++u) {
      const int p = tid + 256 * u, rr = p / (kWgTile / 8), cc = (p % (kWgTile / 8)) * 8;
      const int r = r0 + rr;
      va[u] = r < r_hi ? *reinterpret_cast<const uint4*>(dy + (int64_t)r * ld_dy + c1 + cc) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < NPB; ++u) {
      const int p = tid + 256 * u, rr = p / (WB / 8), cc = (p % (WB / 8)) * 8;
      const int r = r0 + rr;
      vb[u] = r < r_hi ? *reinterpret_cast<const uint4*>(x + (int64_t)r * ld_x + c2 + cc) : make_uint4(0, 0, 0, 0);
    }
  };
  auto stage = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < NPA; ++u) {
      const int p = tid + 256 * u, rr = p / (kWgTile / 8), cc = (p % (kWgTile / 8)) * 8;
      *reinterpret_cast<uint4*>(&sa[buf][rr * PA + cc]) = va[u];
    }
#pragma unroll
    for (int u = 0; u < NPB; ++u) {
      const int p = tid + 256 * u, rr = p / (WB / 8), cc = (p % (WB / 8)) * 8;
      *reinterpret_cast<uint4*>(&sb[buf][rr * PB + cc]) = vb[u];
    }
  };
  f32x4 acc[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) acc[s] = zero4();
  int buf = 0;
  if (r_lo < r_hi) {
    load(r_lo);
    stage(0);
  }
  for (int r0 = r_lo; r0 < r_hi; r0 += kWgRows) {
    __syncthreads();  // step r0 is staged in buf; the other buffer is free
    const bool more = r0 + kWgRows < r_hi;
    if (more) load(r0 + kWgRows);
#pragma unroll
    for (int kc = 0; kc < kWgRows / 32; ++kc) {
      // K slots 8g..8g+7 of a fragment are token rows kc*32 + 8g .. + 7: lanes 4 rho ..
      // 4 rho + 3 of a 16-lane group address row rho of a 4 x 16 block (transpose load)
      const int row = kc * 32 + 8 * g + (j >> 2), col = 4 * (j & 3);
      const uint4 a = ld_tr_pair(&sa[buf][row * PA + wave * 16 + col], 4 * PA);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const uint4 b = ld_tr_pair(&sb[buf][row * PB + s * 16 + col], 4 * PB);
        acc[s] = Mma<bf16>::run(acc[s], a, b);
      }
    }
    if (more) stage(buf ^ 1);
    buf ^= 1;
  }
  // acc[s][i]: output (c1 + 16 wave + 4 g + i, c2 + 16 s + j)
  float* pt = part + (int64_t)blockIdx.z * n1 * n2;
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i) pt[(int64_t)(c1 + wave * 16 + 4 * g + i) * n2 + c2 + s * 16 + j] = acc[s][i];
}

// dW = the chunks' partial tiles added in chunk order (reproducible), rounded once; eight
// chunks' loads in flight per step
__global__ __launch_bounds__(256) void wgrad_sum_kernel(const float* __restrict__ part, int nchunks, int n1, int n2,
                                                        uint16_t* __restrict__ dw, int64_t ld_dw) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t ne = (int64_t)n1 * n2;
  if (e >= ne) return;
  float s = 0.f;
  int c = 0;
  for (; c + 8 <= nchunks; c += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = __builtin_nontemporal_load(part + (c + u) * ne + e);
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  for (; c < nchunks; ++c) s += part[c * ne + e];
  dw[(e / n2) * ld_dw + e % n2] = f32_to_bf16_bits(s);
}

}  // namespace nsa

extern "C" size_t nsa_wgrad_workspace_size(int rows, int n1, int n2) {
  if (rows <= 0 || n1 <= 0 || n2 <= 0 || n1 % nsa::kWgTile || n2 % nsa::kWgTile) return 0;
  const int per = nsa::wgrad_chunk_rows(rows, n1, n2);
  const size_t nchunks = (size_t)((rows + per - 1) / per);
  return nchunks * (size_t)n1 * (size_t)n2 * sizeof(float);
}

extern "C" int nsa_wgrad(const void* dy, int64_t ld_dy, const void* x, int64_t ld_x, int rows, int n1, int n2,
                         void* dw, int64_t ld_dw, int dtype, void* workspace, size_t workspace_bytes,
                         nsa_stream_t stream) {
  using namespace nsa;
  if (dtype != NSA_BF16) return set_error(NSA_ERR_UNSUPPORTED, "nsa_wgrad: bf16 only");
  if (rows < 0 || n1 <= 0 || n2 <= 0 || n1 % kWgTile || n2 % kWgTile)
    return set_error(NSA_ERR_INVALID, "nsa_wgrad: n1 and n2 must be positive multiples of 64, rows >= 0");
  if ((rows > 0 && (!dy || !x)) || !dw) return set_error(NSA_ERR_INVALID, "nsa_wgrad: null pointer");
  if ((uintptr_t)dy % 16 || (uintptr_t)x % 16 || ld_dy % 8 || ld_x % 8 || ld_dy < n1 || ld_x < n2 || ld_dw < n2)
    return set_error(NSA_ERR_LAYOUT, "nsa_wgrad: rows must be 16-byte aligned with unit feature stride");
  hipStream_t st = (hipStream_t)stream;
  if (rows == 0) {
    hipLaunchKernelGGL(wgrad_sum_kernel, dim3((unsigned)(((int64_t)n1 * n2 + 255) / 256)), dim3(256), 0, st,
                       (const float*)nullptr, 0, n1, n2, (uint16_t*)dw, ld_dw);
  } else {
    const size_t need = nsa_wgrad_workspace_size(rows, n1, n2);
    if (!workspace || workspace_bytes < need) {
      char msg[128];
      snprintf(msg, sizeof msg, "nsa_wgrad: workspace %zu bytes < required %zu", workspace_bytes, need);
      return set_error(NSA_ERR_WORKSPACE, msg);
    }
    const int per = wgrad_chunk_rows(rows, n1, n2);
    const int nchunks = (rows + per - 1) / per;
    float* part = reinterpret_cast<float*>(workspace);
    const int wb = wgrad_block_cols(n2);
    const dim3 grid(n1 / kWgTile, n2 / wb, nchunks);
    if (wb == 192)
      hipLaunchKernelGGL(wgrad_partial_kernel<12>, grid, dim3(256), 0, st, (const uint16_t*)dy, ld_dy,
                         (const uint16_t*)x, ld_x, rows, n1, n2, per, part);
    else if (wb == 128)
      hipLaunchKernelGGL(wgrad_partial_kernel<8>, grid, dim3(256), 0, st, (const uint16_t*)dy, ld_dy,
                         (const uint16_t*)x, ld_x, rows, n1, n2, per, part);
    else
      hipLaunchKernelGGL(wgrad_partial_kernel<4>, grid, dim3(256), 0, st, (const uint16_t*)dy, ld_dy,
                         (const uint16_t*)x, ld_x, rows, n1, n2, per, part);
    hipLaunchKernelGGL(wgrad_sum_kernel, dim3((unsigned)(((int64_t)n1 * n2 + 255) / 256)), dim3(256), 0, st,
                       (const float*)part, nchunks, n1, n2, (uint16_t*)dw, ld_dw);
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? NSA_OK : set_error(NSA_ERR_HIP, hipGetErrorString(e));
}
