// Compression-token pooling (the reference's compress_tokens, nsa/kernels.py:2119-2208)
// restructured for the GPU.
//
// Reference: K_cmp[i] = mean_{u<l} W2 relu(W1 [k_{d*i+u} ; E[u]] + b1) + b2,
//            V_cmp[i] = mean_{u<l} v_{d*i+u}.
// Split W1 = [W1k | W1p]: the pre-activation is Y[t] + C[u] with Y = k W1k^T (one GEMM
// over the T tokens instead of over the l/d-times-duplicated blocks) and
// C = E W1p^T + b1 (l x 2dk).  W2 and the mean commute, so
//            K_cmp[i] = W2 R[i] + b2,   R[i] = mean_u relu(Y[d*i+u] + C[u]),
// a GEMM over the n_cmp pooled rows.  The GEMMs and their input gradients stay in torch
// (hipBLASLt), the weight gradients are nsa_wgrad (nsa_wgrad.hip); this file holds the
// HBM-bound middle: R and V_cmp (forward) and dY, dC, dV (backward).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nsa_hip.h"
#include "nsa_device.h"
#include "nsa_kernels.h"

namespace nsa {

// Row of token t of (batch, group) bg: group-major [B,G,T,*] storage (tm = 0) or the
// token-major [B,T,G,*] storage the module's projections produce (tm = 1).
__device__ __forceinline__ int64_t pool_row(int64_t bg, int64_t t, int T_, int G, int tm) {
  return tm ? ((bg / G) * T_ + t) * G + bg % G : bg * T_ + t;
}

template <typename T>
__global__ __launch_bounds__(256) void pool_fwd_kernel(const typename Store<T>::type* __restrict__ Y,
                                                       const typename Store<T>::type* __restrict__ C,
                                                       const typename Store<T>::type* __restrict__ V,
                                                       typename Store<T>::type* __restrict__ R,
                                                       typename Store<T>::type* __restrict__ Vc, int T_, int W, int dv,
                                                       int l, int d, int n_act, int G, int tm) {
  // grid: (n_act, B*G); threads stride over the W + dv channels
  const int i = blockIdx.x;
  const int64_t bg = blockIdx.y;
  const float inv = 1.0f / (float)l;
  const int64_t t0 = (int64_t)i * d;
  for (int c = threadIdx.x; c < W + dv; c += 256) {
    float acc = 0.f;
    if (c < W) {
      for (int u = 0; u < l; ++u) {
        const float y = Elem<T>::to_f32(Y[pool_row(bg, t0 + u, T_, G, tm) * W + c]) + Elem<T>::to_f32(C[(int64_t)u * W + c]);
        acc += y > 0.f ? y : 0.f;
      }
      R[(bg * n_act + i) * W + c] = Elem<T>::from_f32(acc * inv);
    } else {
      const int e = c - W;
      for (int u = 0; u < l; ++u) acc += Elem<T>::to_f32(V[pool_row(bg, t0 + u, T_, G, tm) * dv + e]);
      Vc[(bg * n_act + i) * dv + e] = Elem<T>::from_f32(acc * inv);
    }
  }
}

// dY[t] = (1/l) sum_{blocks i holding t} dR[i] * [Y[t] + C[t - d*i] > 0]
// dV[t] = (1/l) sum_{blocks i holding t} dVc[i]
template <typename T>
__global__ __launch_bounds__(256) void pool_bwd_tok_kernel(const typename Store<T>::type* __restrict__ Y,
                                                           const typename Store<T>::type* __restrict__ C,
                                                           const typename Store<T>::type* __restrict__ dR,
                                                           const typename Store<T>::type* __restrict__ dVc,
                                                           typename Store<T>::type* __restrict__ dY,
                                                           typename Store<T>::type* __restrict__ dV, int T_, int W,
                                                           int dv, int l, int d, int n_act, int G, int tm) {
  const int t = blockIdx.x;
  const int64_t bg = blockIdx.y;
  const float inv = 1.0f / (float)l;
  // blocks i with d*i <= t < d*i + l, 0 <= i < n_act (ascending i)
  int i_lo = t - l + 1 <= 0 ? 0 : (t - l + 1 + d - 1) / d;
  int i_hi = min(t / d, n_act - 1);
  const int64_t row = pool_row(bg, t, T_, G, tm);
  for (int c = threadIdx.x; c < W + dv; c += 256) {
    float acc = 0.f;
    if (c < W) {
      const float y = Elem<T>::to_f32(Y[row * W + c]);
      for (int i = i_lo; i <= i_hi; ++i) {
        const int u = t - d * i;
        if (y + Elem<T>::to_f32(C[(int64_t)u * W + c]) > 0.f)
          acc += Elem<T>::to_f32(dR[(bg * n_act + i) * W + c]);
      }
      dY[row * W + c] = Elem<T>::from_f32(acc * inv);
    } else {
      const int e = c - W;
      for (int i = i_lo; i <= i_hi; ++i) acc += Elem<T>::to_f32(dVc[(bg * n_act + i) * dv + e]);
      dV[row * dv + e] = Elem<T>::from_f32(acc * inv);
    }
  }
}

// dC[u] = (1/l) sum_{b,g,i} dR[b,g,i] * [Y[d*i+u] + C[u] > 0]   (fp32, fixed order)
template <typename T>
__global__ __launch_bounds__(256) void pool_bwd_c_kernel(const typename Store<T>::type* __restrict__ Y,
                                                         const typename Store<T>::type* __restrict__ C,
                                                         const typename Store<T>::type* __restrict__ dR,
                                                         float* __restrict__ dC, int BG, int T_, int W, int l, int d,
                                                         int n_act, int G, int tm) {
  // 64 channels x 4 interleaved block groups per workgroup; the 4 group sums are
  // combined in a fixed order
  __shared__ float part[4][64];
  const int u = blockIdx.y;
  const int cl = threadIdx.x & 63, ig = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + cl;
  float acc = 0.f;
  if (c < W) {
    const float cu = Elem<T>::to_f32(C[(int64_t)u * W + c]);
    for (int64_t bg = 0; bg < BG; ++bg) {
#pragma unroll 4
      for (int i = ig; i < n_act; i += 4) {
        const float y = Elem<T>::to_f32(Y[pool_row(bg, (int64_t)i * d + u, T_, G, tm) * W + c]);
        const float g = Elem<T>::to_f32(dR[(bg * n_act + i) * W + c]);
        acc += (y + cu > 0.f) ? g : 0.f;
      }
    }
  }
  part[ig][cl] = acc;
  __syncthreads();
  if (ig == 0 && c < W) dC[(int64_t)u * W + c] = (((part[0][cl] + part[1][cl]) + part[2][cl]) + part[3][cl]) / (float)l;
}

// Vectorised forms of the two backward kernels for widths that are multiples of a
// 16-byte piece (EPF elements): one thread per piece.
template <typename T>
__device__ __forceinline__ void unpack16(const uint4& v, float* f) {
  if constexpr (sizeof(typename Store<T>::type) == 2) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      f[2 * k] = __uint_as_float(w[k] << 16);
      f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
  } else {
    f[0] = __uint_as_float(v.x);
    f[1] = __uint_as_float(v.y);
    f[2] = __uint_as_float(v.z);
    f[3] = __uint_as_float(v.w);
  }
}
template <typename T>
__device__ __forceinline__ uint4 pack16(const float* f) {
  if constexpr (sizeof(typename Store<T>::type) == 2) {
    return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                      pack_bf16x2(f[6], f[7]));
  } else {
    return make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3]));
  }
}

// dY / dV as pool_bwd_tok_kernel; ppt = (W + dv) / EPF pieces per token, 256 / ppt
// tokens per workgroup (ppt <= 256)
template <typename T>
__global__ __launch_bounds__(256) void pool_bwd_tok_vec_kernel(const typename Store<T>::type* __restrict__ Y,
                                                               const typename Store<T>::type* __restrict__ C,
                                                               const typename Store<T>::type* __restrict__ dR,
                                                               const typename Store<T>::type* __restrict__ dVc,
                                                               typename Store<T>::type* __restrict__ dY,
                                                               typename Store<T>::type* __restrict__ dV, int T_, int W,
                                                               int dv, int l, int d, int n_act, int ppt, int G, int tm) {
  constexpr int EPF = 16 / sizeof(typename Store<T>::type);
  const int tpw = 256 / ppt;
  const int t = blockIdx.x * tpw + threadIdx.x / ppt;
  const int pc = threadIdx.x % ppt;
  if (threadIdx.x >= tpw * ppt || t >= T_) return;
  const int64_t bg = blockIdx.y;
  const float inv = 1.0f / (float)l;
  const int i_lo = t - l + 1 <= 0 ? 0 : (t - l + 1 + d - 1) / d;
  const int i_hi = min(t / d, n_act - 1);
  const int64_t row = pool_row(bg, t, T_, G, tm);
  float acc[EPF], x[EPF];
#pragma unroll
  for (int k = 0; k < EPF; ++k) acc[k] = 0.f;
  const int c = pc * EPF;
  if (c < W) {
    float y[EPF], cu[EPF];
    unpack16<T>(*reinterpret_cast<const uint4*>(Y + row * W + c), y);
    for (int i = i_lo; i <= i_hi; ++i) {
      const int u = t - d * i;
      unpack16<T>(*reinterpret_cast<const uint4*>(C + (int64_t)u * W + c), cu);
      unpack16<T>(*reinterpret_cast<const uint4*>(dR + (bg * n_act + i) * W + c), x);
#pragma unroll
      for (int k = 0; k < EPF; ++k)
        if (y[k] + cu[k] > 0.f) acc[k] += x[k];
    }
#pragma unroll
    for (int k = 0; k < EPF; ++k) acc[k] *= inv;
    *reinterpret_cast<uint4*>(dY + row * W + c) = pack16<T>(acc);
  } else {
    const int e = c - W;
    for (int i = i_lo; i <= i_hi; ++i) {
      unpack16<T>(*reinterpret_cast<const uint4*>(dVc + (bg * n_act + i) * dv + e), x);
#pragma unroll
      for (int k = 0; k < EPF; ++k) acc[k] += x[k];
    }
#pragma unroll
    for (int k = 0; k < EPF; ++k) acc[k] *= inv;
    *reinterpret_cast<uint4*>(dV + row * dv + e) = pack16<T>(acc);
  }
}

// dC as pool_bwd_c_kernel: workgroup = (64 channels, u); its 1024 threads are 64 / EPF
// piece columns x 1024 / (64 / EPF) interleaved groups of the (b, g, i) rows, whose partial sums
// are combined in group order.
template <typename T>
__global__ __launch_bounds__(1024) void pool_bwd_c_vec_kernel(const typename Store<T>::type* __restrict__ Y,
                                                              const typename Store<T>::type* __restrict__ C,
                                                              const typename Store<T>::type* __restrict__ dR,
                                                              float* __restrict__ dC, int BG, int T_, int W, int l,
                                                              int d, int n_act, int G, int tm) {
  constexpr int EPF = 16 / sizeof(typename Store<T>::type);
  constexpr int NPC = 64 / EPF;             // piece columns per workgroup
  constexpr int NG = 1024 / NPC;            // row groups
  __shared__ float part[NG][64 + 1];
  const int u = blockIdx.y;
  const int pcl = threadIdx.x % NPC, grp = threadIdx.x / NPC;
  const int c = blockIdx.x * 64 + pcl * EPF;
  float acc[EPF];
#pragma unroll
  for (int k = 0; k < EPF; ++k) acc[k] = 0.f;
  if (c < W) {
    float cu[EPF], y[EPF], g[EPF];
    unpack16<T>(*reinterpret_cast<const uint4*>(C + (int64_t)u * W + c), cu);
    const int64_t nrows = (int64_t)BG * n_act;
    for (int64_t q = grp; q < nrows; q += NG) {
      const int64_t bg = q / n_act;
      const int i = (int)(q % n_act);
      unpack16<T>(*reinterpret_cast<const uint4*>(Y + pool_row(bg, (int64_t)i * d + u, T_, G, tm) * W + c), y);
      unpack16<T>(*reinterpret_cast<const uint4*>(dR + q * W + c), g);
#pragma unroll
      for (int k = 0; k < EPF; ++k)
        if (y[k] + cu[k] > 0.f) acc[k] += g[k];
    }
  }
#pragma unroll
  for (int k = 0; k < EPF; ++k) part[grp][pcl * EPF + k] = acc[k];
  __syncthreads();
  if (threadIdx.x < 64) {
    const int cc = blockIdx.x * 64 + threadIdx.x;
    float s = 0.f;
    for (int gi = 0; gi < NG; ++gi) s += part[gi][threadIdx.x];
    if (cc < W) dC[(int64_t)u * W + cc] = s / (float)l;
  }
}

// R / V_cmp as pool_fwd_kernel, one thread per 16-byte piece of a block's W + dv
// channels; 256 / ppt blocks per workgroup
template <typename T>
__global__ __launch_bounds__(256) void pool_fwd_vec_kernel(const typename Store<T>::type* __restrict__ Y,
                                                           const typename Store<T>::type* __restrict__ C,
                                                           const typename Store<T>::type* __restrict__ V,
                                                           typename Store<T>::type* __restrict__ R,
                                                           typename Store<T>::type* __restrict__ Vc, int T_, int W,
                                                           int dv, int l, int d, int n_act, int ppt, int G, int tm) {
  constexpr int EPF = 16 / sizeof(typename Store<T>::type);
  const int bpw = 256 / ppt;
  const int i = blockIdx.x * bpw + threadIdx.x / ppt;
  const int pc = threadIdx.x % ppt;
  if (threadIdx.x >= bpw * ppt || i >= n_act) return;
  const int64_t bg = blockIdx.y;
  const float inv = 1.0f / (float)l;
  const int64_t t0 = (int64_t)i * d;
  float acc[EPF], x[EPF];
#pragma unroll
  for (int k = 0; k < EPF; ++k) acc[k] = 0.f;
  const int c = pc * EPF;
  if (c < W) {
    float cu[EPF];
#pragma unroll 8
    for (int u = 0; u < l; ++u) {
      unpack16<T>(*reinterpret_cast<const uint4*>(Y + pool_row(bg, t0 + u, T_, G, tm) * W + c), x);
      unpack16<T>(*reinterpret_cast<const uint4*>(C + (int64_t)u * W + c), cu);
#pragma unroll
      for (int k = 0; k < EPF; ++k) {
        const float y = x[k] + cu[k];
        acc[k] += y > 0.f ? y : 0.f;
      }
    }
#pragma unroll
    for (int k = 0; k < EPF; ++k) acc[k] *= inv;
    *reinterpret_cast<uint4*>(R + (bg * n_act + i) * W + c) = pack16<T>(acc);
  } else {
    const int e = c - W;
#pragma unroll 8
    for (int u = 0; u < l; ++u) {
      unpack16<T>(*reinterpret_cast<const uint4*>(V + pool_row(bg, t0 + u, T_, G, tm) * dv + e), x);
#pragma unroll
      for (int k = 0; k < EPF; ++k) acc[k] += x[k];
    }
#pragma unroll
    for (int k = 0; k < EPF; ++k) acc[k] *= inv;
    *reinterpret_cast<uint4*>(Vc + (bg * n_act + i) * dv + e) = pack16<T>(acc);
  }
}

}  // namespace nsa

using namespace nsa;

// All tensors compact (row-major): Y [B,G,T,W] (token_major: [B,T,G,W]), C [l,W],
// V [B,G,T,dv] (token_major: [B,T,G,dv]), R [B,G,n_act,W], Vc [B,G,n_act,dv].
extern "C" int nsa_compress_pool_fwd(const void* Y, const void* C, const void* V, void* R, void* Vc, int Z, int G,
                                     int n_ctx, int width, int head_dim_v, int l, int d, int n_act, int token_major,
                                     int dtype, nsa_stream_t stream) {
  const int tm = token_major ? 1 : 0;
  if (dtype != NSA_F32 && dtype != NSA_BF16) return set_error(NSA_ERR_INVALID, "dtype not supported");
  if (Z <= 0 || G <= 0 || l <= 0 || d <= 0 || n_act < 0 || width <= 0 || head_dim_v <= 0)
    return set_error(NSA_ERR_INVALID, "bad shape");
  if (n_act > 0 && (int64_t)(n_act - 1) * d + l > n_ctx) return set_error(NSA_ERR_INVALID, "blocks exceed n_ctx");
  if (n_act == 0) return NSA_OK;
  TimingScope ts(kIdPoolFwd, (hipStream_t)stream);
  dim3 grid(n_act, Z * G);
  hipStream_t st = (hipStream_t)stream;
  {
    const int epf = dtype == NSA_F32 ? 4 : 8;
    const int ppt = (width + head_dim_v) / epf;
    const bool al = ((uintptr_t)Y | (uintptr_t)C | (uintptr_t)V | (uintptr_t)R | (uintptr_t)Vc) % 16 == 0;
    if (al && width % epf == 0 && head_dim_v % epf == 0 && ppt <= 256) {
      const int bpw = 256 / ppt;
      dim3 gv((n_act + bpw - 1) / bpw, Z * G);
      if (dtype == NSA_F32)
        hipLaunchKernelGGL(pool_fwd_vec_kernel<float>, gv, dim3(256), 0, st, (const float*)Y, (const float*)C,
                           (const float*)V, (float*)R, (float*)Vc, n_ctx, width, head_dim_v, l, d, n_act, ppt, G, tm);
      else
        hipLaunchKernelGGL(pool_fwd_vec_kernel<bf16>, gv, dim3(256), 0, st, (const uint16_t*)Y, (const uint16_t*)C,
                           (const uint16_t*)V, (uint16_t*)R, (uint16_t*)Vc, n_ctx, width, head_dim_v, l, d, n_act,
                           ppt, G, tm);
      hipError_t e = hipGetLastError();
      return e == hipSuccess ? NSA_OK : set_error(NSA_ERR_HIP, hipGetErrorString(e));
    }
  }
  if (dtype == NSA_F32)
    hipLaunchKernelGGL(pool_fwd_kernel<float>, grid, dim3(256), 0, st, (const float*)Y, (const float*)C,
                       (const float*)V, (float*)R, (float*)Vc, n_ctx, width, head_dim_v, l, d, n_act, G, tm);
  else
    hipLaunchKernelGGL(pool_fwd_kernel<bf16>, grid, dim3(256), 0, st, (const uint16_t*)Y, (const uint16_t*)C,
                       (const uint16_t*)V, (uint16_t*)R, (uint16_t*)Vc, n_ctx, width, head_dim_v, l, d, n_act, G, tm);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? NSA_OK : set_error(NSA_ERR_HIP, hipGetErrorString(e));
}

// dY [B,G,T,W] and dV [B,G,T,dv] (token_major: [B,T,G,*], as Y and V) are overwritten
// (element type = dtype); dC [l,W] fp32.
extern "C" int nsa_compress_pool_bwd(const void* Y, const void* C, const void* dR, const void* dVc, void* dY,
                                     float* dC, void* dV, int Z, int G, int n_ctx, int width, int head_dim_v, int l,
                                     int d, int n_act, int token_major, int dtype, nsa_stream_t stream) {
  const int tm = token_major ? 1 : 0;
  if (dtype != NSA_F32 && dtype != NSA_BF16) return set_error(NSA_ERR_INVALID, "dtype not supported");
  if (Z <= 0 || G <= 0 || l <= 0 || d <= 0 || n_act < 0 || width <= 0 || head_dim_v <= 0)
    return set_error(NSA_ERR_INVALID, "bad shape");
  if (n_act > 0 && (int64_t)(n_act - 1) * d + l > n_ctx) return set_error(NSA_ERR_INVALID, "blocks exceed n_ctx");
  if (n_ctx == 0) return NSA_OK;
  hipStream_t st = (hipStream_t)stream;
  TimingScope ts(kIdPoolBwd, (hipStream_t)stream);
  dim3 gt(n_ctx, Z * G), gc((width + 63) / 64, l);
  {
    const int epf = dtype == NSA_F32 ? 4 : 8;
    const int ppt = (width + head_dim_v) / epf;
    const bool al = ((uintptr_t)Y | (uintptr_t)C | (uintptr_t)dR | (uintptr_t)dVc | (uintptr_t)dY | (uintptr_t)dV) % 16 == 0;
    if (al && width % epf == 0 && head_dim_v % epf == 0 && ppt <= 256) {
      const int tpw = 256 / ppt;
      dim3 gv((n_ctx + tpw - 1) / tpw, Z * G);
      if (dtype == NSA_F32) {
        hipLaunchKernelGGL(pool_bwd_tok_vec_kernel<float>, gv, dim3(256), 0, st, (const float*)Y, (const float*)C,
                           (const float*)dR, (const float*)dVc, (float*)dY, (float*)dV, n_ctx, width, head_dim_v, l,
                           d, n_act, ppt, G, tm);
        hipLaunchKernelGGL(pool_bwd_c_vec_kernel<float>, gc, dim3(1024), 0, st, (const float*)Y, (const float*)C,
                           (const float*)dR, dC, Z * G, n_ctx, width, l, d, n_act, G, tm);
      } else {
        hipLaunchKernelGGL(pool_bwd_tok_vec_kernel<bf16>, gv, dim3(256), 0, st, (const uint16_t*)Y,
                           (const uint16_t*)C, (const uint16_t*)dR, (const uint16_t*)dVc, (uint16_t*)dY,
                           (uint16_t*)dV, n_ctx, width, head_dim_v, l, d, n_act, ppt, G, tm);
        hipLaunchKernelGGL(pool_bwd_c_vec_kernel<bf16>, gc, dim3(1024), 0, st, (const uint16_t*)Y,
                           (const uint16_t*)C, (const uint16_t*)dR, dC, Z * G, n_ctx, width, l, d, n_act, G, tm);
      }
      hipError_t e = hipGetLastError();
      return e == hipSuccess ? NSA_OK : set_error(NSA_ERR_HIP, hipGetErrorString(e));
    }
  }
  if (dtype == NSA_F32) {
    hipLaunchKernelGGL(pool_bwd_tok_kernel<float>, gt, dim3(256), 0, st, (const float*)Y, (const float*)C,
                       (const float*)dR, (const float*)dVc, (float*)dY, (float*)dV, n_ctx, width, head_dim_v, l, d,
                       n_act, G, tm);
    hipLaunchKernelGGL(pool_bwd_c_kernel<float>, gc, dim3(256), 0, st, (const float*)Y, (const float*)C,
                       (const float*)dR, dC, Z * G, n_ctx, width, l, d, n_act, G, tm);
  } else {
    hipLaunchKernelGGL(pool_bwd_tok_kernel<bf16>, gt, dim3(256), 0, st, (const uint16_t*)Y, (const uint16_t*)C,
                       (const uint16_t*)dR, (const uint16_t*)dVc, (uint16_t*)dY, (uint16_t*)dV, n_ctx, width,
                       head_dim_v, l, d, n_act, G, tm);
    hipLaunchKernelGGL(pool_bwd_c_kernel<bf16>, gc, dim3(256), 0, st, (const uint16_t*)Y, (const uint16_t*)C,
                       (const uint16_t*)dR, dC, Z * G, n_ctx, width, l, d, n_act, G, tm);
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? NSA_OK : set_error(NSA_ERR_HIP, hipGetErrorString(e));
}
