// Compression-token pooling (the reference's compress_tokens, nsa/kernels.py:2119-2208)
// restructured for the GPU.
//
// Reference: K_cmp[i] = mean_{u<l} W2 relu(W1 [k_{d*i+u} ; E[u]] + b1) + b2,
//            V_cmp[i] = mean_{u<l} v_{d*i+u}.
// Split W1 = [W1k | W1p]: the pre-activation is Y[t] + C[u] with Y = k W1k^T (one GEMM
// over the T tokens instead of over the l/d-times-duplicated blocks) and
// C = E W1p^T + b1 (l x 2dk).  W2 and the mean commute, so
//            K_cmp[i] = W2 R[i] + b2,   R[i] = mean_u relu(Y[d*i+u] + C[u]),
// a GEMM over the n_cmp pooled rows.  The GEMMs stay in torch (hipBLASLt); this file
// holds the HBM-bound middle: R and V_cmp (forward) and dY, dC, dV (backward).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nsa_hip.h"
#include "nsa_device.h"
#include "nsa_kernels.h"

namespace nsa {

template <typename T>
__global__ __launch_bounds__(256) void pool_fwd_kernel(const typename Store<T>::type* __restrict__ Y,
                                                       const typename Store<T>::type* __restrict__ C,
                                                       const typename Store<T>::type* __restrict__ V,
                                                       typename Store<T>::type* __restrict__ R,
                                                       typename Store<T>::type* __restrict__ Vc, int T_, int W, int dv,
                                                       int l, int d, int n_act) {
  // grid: (n_act, B*G); threads stride over the W + dv channels
  const int i = blockIdx.x;
  const int64_t bg = blockIdx.y;
  const float inv = 1.0f / (float)l;
  const int64_t row0 = bg * T_ + (int64_t)i * d;
  for (int c = threadIdx.x; c < W + dv; c += 256) {
    float acc = 0.f;
    if (c < W) {
      for (int u = 0; u < l; ++u) {
        const float y = Elem<T>::to_f32(Y[(row0 + u) * W + c]) + Elem<T>::to_f32(C[(int64_t)u * W + c]);
        acc += y > 0.f ? y : 0.f;
      }
      R[(bg * n_act + i) * W + c] = Elem<T>::from_f32(acc * inv);
    } else {
      const int e = c - W;
      for (int u = 0; u < l; ++u) acc += Elem<T>::to_f32(V[(row0 + u) * dv + e]);
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
                                                           int dv, int l, int d, int n_act) {
  const int t = blockIdx.x;
  const int64_t bg = blockIdx.y;
  const float inv = 1.0f / (float)l;
  // blocks i with d*i <= t < d*i + l, 0 <= i < n_act (ascending i)
  int i_lo = t - l + 1 <= 0 ? 0 : (t - l + 1 + d - 1) / d;
  int i_hi = min(t / d, n_act - 1);
  const int64_t row = bg * T_ + t;
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
                                                         int n_act) {
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
        const float y = Elem<T>::to_f32(Y[(bg * T_ + (int64_t)i * d + u) * W + c]);
        const float g = Elem<T>::to_f32(dR[(bg * n_act + i) * W + c]);
        acc += (y + cu > 0.f) ? g : 0.f;
      }
    }
  }
  part[ig][cl] = acc;
  __syncthreads();
  if (ig == 0 && c < W) dC[(int64_t)u * W + c] = (((part[0][cl] + part[1][cl]) + part[2][cl]) + part[3][cl]) / (float)l;
}

}  // namespace nsa

using namespace nsa;

// All tensors compact (row-major): Y [B,G,T,W], C [l,W], V [B,G,T,dv],
// R [B,G,n_act,W], Vc [B,G,n_act,dv].
extern "C" int nsa_compress_pool_fwd(const void* Y, const void* C, const void* V, void* R, void* Vc, int Z, int G,
                                     int n_ctx, int width, int head_dim_v, int l, int d, int n_act, int dtype,
                                     nsa_stream_t stream) {
  if (dtype != NSA_F32 && dtype != NSA_BF16) return set_error(NSA_ERR_INVALID, "dtype not supported");
  if (Z <= 0 || G <= 0 || l <= 0 || d <= 0 || n_act < 0 || width <= 0 || head_dim_v <= 0)
    return set_error(NSA_ERR_INVALID, "bad shape");
  if (n_act > 0 && (int64_t)(n_act - 1) * d + l > n_ctx) return set_error(NSA_ERR_INVALID, "blocks exceed n_ctx");
  if (n_act == 0) return NSA_OK;
  TimingScope ts(kIdPoolFwd, (hipStream_t)stream);
  dim3 grid(n_act, Z * G);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == NSA_F32)
    hipLaunchKernelGGL(pool_fwd_kernel<float>, grid, dim3(256), 0, st, (const float*)Y, (const float*)C,
                       (const float*)V, (float*)R, (float*)Vc, n_ctx, width, head_dim_v, l, d, n_act);
  else
    hipLaunchKernelGGL(pool_fwd_kernel<bf16>, grid, dim3(256), 0, st, (const uint16_t*)Y, (const uint16_t*)C,
                       (const uint16_t*)V, (uint16_t*)R, (uint16_t*)Vc, n_ctx, width, head_dim_v, l, d, n_act);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? NSA_OK : set_error(NSA_ERR_HIP, hipGetErrorString(e));
}

// dY [B,G,T,W] and dV [B,G,T,dv] are overwritten (element type = dtype); dC [l,W] fp32.
extern "C" int nsa_compress_pool_bwd(const void* Y, const void* C, const void* dR, const void* dVc, void* dY,
                                     float* dC, void* dV, int Z, int G, int n_ctx, int width, int head_dim_v, int l,
                                     int d, int n_act, int dtype, nsa_stream_t stream) {
  if (dtype != NSA_F32 && dtype != NSA_BF16) return set_error(NSA_ERR_INVALID, "dtype not supported");
  if (Z <= 0 || G <= 0 || l <= 0 || d <= 0 || n_act < 0 || width <= 0 || head_dim_v <= 0)
    return set_error(NSA_ERR_INVALID, "bad shape");
  if (n_act > 0 && (int64_t)(n_act - 1) * d + l > n_ctx) return set_error(NSA_ERR_INVALID, "blocks exceed n_ctx");
  if (n_ctx == 0) return NSA_OK;
  hipStream_t st = (hipStream_t)stream;
  TimingScope ts(kIdPoolBwd, (hipStream_t)stream);
  dim3 gt(n_ctx, Z * G), gc((width + 63) / 64, l);
  if (dtype == NSA_F32) {
    hipLaunchKernelGGL(pool_bwd_tok_kernel<float>, gt, dim3(256), 0, st, (const float*)Y, (const float*)C,
                       (const float*)dR, (const float*)dVc, (float*)dY, (float*)dV, n_ctx, width, head_dim_v, l, d,
                       n_act);
    hipLaunchKernelGGL(pool_bwd_c_kernel<float>, gc, dim3(256), 0, st, (const float*)Y, (const float*)C,
                       (const float*)dR, dC, Z * G, n_ctx, width, l, d, n_act);
  } else {
    hipLaunchKernelGGL(pool_bwd_tok_kernel<bf16>, gt, dim3(256), 0, st, (const uint16_t*)Y, (const uint16_t*)C,
                       (const uint16_t*)dR, (const uint16_t*)dVc, (uint16_t*)dY, (uint16_t*)dV, n_ctx, width,
                       head_dim_v, l, d, n_act);
    hipLaunchKernelGGL(pool_bwd_c_kernel<bf16>, gc, dim3(256), 0, st, (const uint16_t*)Y, (const uint16_t*)C,
                       (const uint16_t*)dR, dC, Z * G, n_ctx, width, l, d, n_act);
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? NSA_OK : set_error(NSA_ERR_HIP, hipGetErrorString(e));
}
