// Gated mix of the three branch outputs (reference nsa/kernels.py NSAAttention.forward:
// o = o_cmp * g[...,0] + o_sel * g[...,1] + o_win * g[...,2]) and its backward, fused:
// one pass over the outputs instead of a chain of broadcast elementwise kernels.  The
// gate activation (reference nsa/kernels.py:2429-2440: sigmoid, or softmax over the
// three gates) can be applied to raw gate logits z in the same pass (gate_act):
//   forward : g = act(z), out = sum_k g_k o_k             (fp32 sum, rounded once)
//   backward: dO_k = g_k dout,  dg_k = sum_d dout . o_k   (fp32), returned as the
//             gradient of the kernel's gate input: dg (act = none), dg_k g_k (1 - g_k)
//             (sigmoid), g_k (dg_k - sum_j g_j dg_j) (softmax)
// Rows are (b, h, t); LPR lanes share a row and read 16-byte pieces of it.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/nsa_hip.h"
#include "nsa_device.h"
#include "nsa_kernels.h"

namespace nsa {

struct MixArgs {
  const void* o[3];
  int64_t so_b, so_h, so_t;
  const void* g;
  int64_t sg_b, sg_h, sg_t, sg_k;
  void* out;  // forward output, or backward dout (read)
  int64_t sx_b, sx_h, sx_t;
  void* dO[3];  // backward: contiguous [B,H,T,dv]
  float* dg;    // backward: contiguous [B,H,T,3]
  float* delta; // backward, optional: contiguous [3][B,H,T], delta_k = g_k dg_k
  int B, H, T, dv;
  int act;  // gate activation applied to the gate input: 0 none, 1 sigmoid, 2 softmax
};

template <typename S>
__device__ __forceinline__ float ld1(const S* p);
template <> __device__ __forceinline__ float ld1<float>(const float* p) { return *p; }
template <> __device__ __forceinline__ float ld1<uint16_t>(const uint16_t* p) { return bf16_bits_to_f32(*p); }

template <typename S>
__device__ __forceinline__ void unpack_piece(const uint4& v, float* f) {
  if constexpr (sizeof(S) == 4) {
    f[0] = __uint_as_float(v.x);
    f[1] = __uint_as_float(v.y);
    f[2] = __uint_as_float(v.z);
    f[3] = __uint_as_float(v.w);
  } else {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      f[2 * u] = __uint_as_float(w[u] << 16);
      f[2 * u + 1] = __uint_as_float(w[u] & 0xffff0000u);
    }
  }
}
template <typename S>
__device__ __forceinline__ uint4 pack_piece(const float* f) {
  if constexpr (sizeof(S) == 4) {
    return make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3]));
  } else {
    return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                      pack_bf16x2(f[6], f[7]));
  }
}

// the gates g_k = act(z_k) of one row: z (none), sigmoid, or softmax over the three
__device__ __forceinline__ void gate_act3(int act, float& g0, float& g1, float& g2) {
  if (act == 1) {
    g0 = 1.f / (1.f + __expf(-g0));
    g1 = 1.f / (1.f + __expf(-g1));
    g2 = 1.f / (1.f + __expf(-g2));
  } else if (act == 2) {
    const float m = fmaxf(g0, fmaxf(g1, g2));
    const float e0 = __expf(g0 - m), e1 = __expf(g1 - m), e2 = __expf(g2 - m);
    const float inv = 1.f / (e0 + e1 + e2);
    g0 = e0 * inv;
    g1 = e1 * inv;
    g2 = e2 * inv;
  }
}

// gradient of the gate input z from the gates g and dg_k = d loss / d g_k (in place on dg)
__device__ __forceinline__ void gate_act3_grad(int act, float g0, float g1, float g2, float& d0, float& d1,
                                               float& d2) {
  if (act == 1) {
    d0 = d0 * g0 * (1.f - g0);
    d1 = d1 * g1 * (1.f - g1);
    d2 = d2 * g2 * (1.f - g2);
  } else if (act == 2) {
    const float s = g0 * d0 + g1 * d1 + g2 * d2;
    d0 = g0 * (d0 - s);
    d1 = g1 * (d1 - s);
    d2 = g2 * (d2 - s);
  }
}

template <typename S, bool BWD>
__global__ __launch_bounds__(256) void gate_mix_kernel(MixArgs a, int lpr_log2) {
  constexpr int EPF = 16 / sizeof(S);
  const int lpr = 1 << lpr_log2;
  const int sub = threadIdx.x & (lpr - 1);
  const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> lpr_log2;
  const int64_t nrows = (int64_t)a.B * a.H * a.T;
  const bool valid = row < nrows;
  const int64_t rr = valid ? row : nrows - 1;
  const int t = rr % a.T;
  const int h = (rr / a.T) % a.H;
  const int b = rr / ((int64_t)a.T * a.H);
  const int64_t ooff = b * a.so_b + h * a.so_h + (int64_t)t * a.so_t;
  const int64_t xoff = b * a.sx_b + h * a.sx_h + (int64_t)t * a.sx_t;
  const S* gp = reinterpret_cast<const S*>(a.g) + b * a.sg_b + h * a.sg_h + (int64_t)t * a.sg_t;
  float g0 = ld1<S>(gp), g1 = ld1<S>(gp + a.sg_k), g2 = ld1<S>(gp + 2 * a.sg_k);
  gate_act3(a.act, g0, g1, g2);
  float dg0 = 0.f, dg1 = 0.f, dg2 = 0.f;
  for (int e = sub * EPF; e < a.dv; e += lpr * EPF) {
    float o0[EPF], o1[EPF], o2[EPF];
    unpack_piece<S>(*reinterpret_cast<const uint4*>(reinterpret_cast<const S*>(a.o[0]) + ooff + e), o0);
    unpack_piece<S>(*reinterpret_cast<const uint4*>(reinterpret_cast<const S*>(a.o[1]) + ooff + e), o1);
    unpack_piece<S>(*reinterpret_cast<const uint4*>(reinterpret_cast<const S*>(a.o[2]) + ooff + e), o2);
    if constexpr (!BWD) {
      float r[EPF];
#pragma unroll
      for (int u = 0; u < EPF; ++u) r[u] = g0 * o0[u] + g1 * o1[u] + g2 * o2[u];
      if (valid) *reinterpret_cast<uint4*>(reinterpret_cast<S*>(a.out) + xoff + e) = pack_piece<S>(r);
    } else {
      float x[EPF], d0[EPF], d1[EPF], d2[EPF];
      unpack_piece<S>(*reinterpret_cast<const uint4*>(reinterpret_cast<const S*>(a.out) + xoff + e), x);
#pragma unroll
      for (int u = 0; u < EPF; ++u) {
        d0[u] = g0 * x[u];
        d1[u] = g1 * x[u];
        d2[u] = g2 * x[u];
        dg0 += x[u] * o0[u];
        dg1 += x[u] * o1[u];
        dg2 += x[u] * o2[u];
      }
      if (valid) {
        const int64_t coff = rr * a.dv + e;
        *reinterpret_cast<uint4*>(reinterpret_cast<S*>(a.dO[0]) + coff) = pack_piece<S>(d0);
        *reinterpret_cast<uint4*>(reinterpret_cast<S*>(a.dO[1]) + coff) = pack_piece<S>(d1);
        *reinterpret_cast<uint4*>(reinterpret_cast<S*>(a.dO[2]) + coff) = pack_piece<S>(d2);
      }
    }
  }
  if constexpr (BWD) {
    for (int off = lpr >> 1; off > 0; off >>= 1) {
      dg0 += __shfl_xor(dg0, off);
      dg1 += __shfl_xor(dg1, off);
      dg2 += __shfl_xor(dg2, off);
    }
    if (valid && sub == 0) {
      if (a.delta) {  // sum_d o_k (g_k dout): the branch backwards' row sums
        a.delta[rr] = g0 * dg0;
        a.delta[nrows + rr] = g1 * dg1;
        a.delta[2 * nrows + rr] = g2 * dg2;
      }
      float z0 = dg0, z1 = dg1, z2 = dg2;  // gradient of the gate input
      gate_act3_grad(a.act, g0, g1, g2, z0, z1, z2);
      a.dg[rr * 3 + 0] = z0;
      a.dg[rr * 3 + 1] = z1;
      a.dg[rr * 3 + 2] = z2;
    }
  }
}

// Gate activation alone (the fused mix path, whose mix runs in the sliding-window
// epilogue): forward z [B,H,T,3] (any strides, fp32 / bf16) -> g [3][B*H*T] fp32;
// backward g and r_k = sum_d dout . o_k ([3][B*H*T] fp32) -> dz [B,H,T,3] (any strides,
// fp32 / bf16).  One thread per (b, h, t) row.
template <typename S, bool BWD>
__global__ __launch_bounds__(256) void gate_act_kernel(const void* zin, float* g, const float* r, void* dz,
                                                       int64_t s_b, int64_t s_h, int64_t s_t, int64_t s_k, int H,
                                                       int T, int64_t nrows, int act) {
  const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (row >= nrows) return;
  const int t = row % T;
  const int h = (row / T) % H;
  const int64_t b = row / ((int64_t)T * H);
  const int64_t off = b * s_b + h * s_h + (int64_t)t * s_t;
  if constexpr (!BWD) {
    const S* zp = reinterpret_cast<const S*>(zin) + off;
    float g0 = ld1<S>(zp), g1 = ld1<S>(zp + s_k), g2 = ld1<S>(zp + 2 * s_k);
    gate_act3(act, g0, g1, g2);
    g[row] = g0;
    g[nrows + row] = g1;
    g[2 * nrows + row] = g2;
  } else {
    const float g0 = g[row], g1 = g[nrows + row], g2 = g[2 * nrows + row];
    float d0 = r[row], d1 = r[nrows + row], d2 = r[2 * nrows + row];
    gate_act3_grad(act, g0, g1, g2, d0, d1, d2);
    S* zp = reinterpret_cast<S*>(dz) + off;
    if constexpr (sizeof(S) == 4) {
      zp[0] = d0;
      zp[s_k] = d1;
      zp[2 * s_k] = d2;
    } else {
      zp[0] = f32_to_bf16_bits(d0);
      zp[s_k] = f32_to_bf16_bits(d1);
      zp[2 * s_k] = f32_to_bf16_bits(d2);
    }
  }
}

template <bool BWD>
static int launch_gate_act(int dtype, const void* z, float* g, const float* r, void* dz, int64_t s_b, int64_t s_h,
                           int64_t s_t, int64_t s_k, int B, int H, int T, int act, hipStream_t st) {
  if (dtype != NSA_F32 && dtype != NSA_BF16) return set_error(NSA_ERR_INVALID, "dtype not supported");
  if (B < 0 || H < 0 || T < 0) return set_error(NSA_ERR_INVALID, "bad shape");
  if (act < 0 || act > 2) return set_error(NSA_ERR_INVALID, "gate_act must be 0, 1 or 2");
  const int64_t nrows = (int64_t)B * H * T;
  if (nrows == 0) return NSA_OK;
  const dim3 grid((unsigned)((nrows + 255) / 256));
  if (dtype == NSA_F32)
    hipLaunchKernelGGL((gate_act_kernel<float, BWD>), grid, dim3(256), 0, st, z, g, r, dz, s_b, s_h, s_t, s_k, H, T,
                       nrows, act);
  else
    hipLaunchKernelGGL((gate_act_kernel<uint16_t, BWD>), grid, dim3(256), 0, st, z, g, r, dz, s_b, s_h, s_t, s_k, H,
                       T, nrows, act);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? NSA_OK : set_error(NSA_ERR_HIP, hipGetErrorString(e));
}

template <bool BWD>
static int launch_mix(int dtype, const MixArgs& a, hipStream_t st) {
  const int64_t nrows = (int64_t)a.B * a.H * a.T;
  if (nrows == 0) return NSA_OK;
  const int pieces = a.dv / (dtype == NSA_F32 ? 4 : 8);
  int lg = 0;
  while ((1 << lg) < pieces && lg < 6) ++lg;
  const int64_t rows_per_wg = 256 >> lg;
  dim3 grid((unsigned)((nrows + rows_per_wg - 1) / rows_per_wg));
  if (dtype == NSA_F32)
    hipLaunchKernelGGL((gate_mix_kernel<float, BWD>), grid, dim3(256), 0, st, a, lg);
  else
    hipLaunchKernelGGL((gate_mix_kernel<uint16_t, BWD>), grid, dim3(256), 0, st, a, lg);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? NSA_OK : set_error(NSA_ERR_HIP, hipGetErrorString(e));
}

static int check_mix(int dtype, int B, int H, int T, int dv, const void* const* ptrs, int n) {
  if (dtype != NSA_F32 && dtype != NSA_BF16) return set_error(NSA_ERR_INVALID, "dtype not supported");
  if (B < 0 || H < 0 || T < 0 || dv <= 0) return set_error(NSA_ERR_INVALID, "bad shape");
  const int epf = dtype == NSA_F32 ? 4 : 8;
  if (dv % epf) return set_error(NSA_ERR_LAYOUT, "head_dim_v must fill 16-byte pieces");
  for (int i = 0; i < n; ++i)
    if (((uintptr_t)ptrs[i]) % 16) return set_error(NSA_ERR_LAYOUT, "branch outputs need 16-byte aligned rows");
  return NSA_OK;
}

}  // namespace nsa

extern "C" int nsa_gate_mix_fwd(const void* o_cmp, const void* o_sel, const void* o_win, int64_t so_b, int64_t so_h,
                                int64_t so_t, const void* gates, int64_t sg_b, int64_t sg_h, int64_t sg_t,
                                int64_t sg_k, void* out, int64_t sout_b, int64_t sout_h, int64_t sout_t, int B, int H,
                                int T, int dv, int gate_act, int dtype, nsa_stream_t stream) {
  using namespace nsa;
  const void* ptrs[4] = {o_cmp, o_sel, o_win, out};
  if (int rc = check_mix(dtype, B, H, T, dv, ptrs, 4)) return rc;
  if (gate_act < 0 || gate_act > 2) return set_error(NSA_ERR_INVALID, "gate_act must be 0, 1 or 2");
  const int esz = dtype == NSA_F32 ? 4 : 2;
  if ((so_t * esz) % 16 || (so_h * esz) % 16 || (sout_t * esz) % 16 || (sout_h * esz) % 16)
    return set_error(NSA_ERR_LAYOUT, "rows must be 16-byte aligned");
  MixArgs a{};
  a.o[0] = o_cmp;
  a.o[1] = o_sel;
  a.o[2] = o_win;
  a.so_b = so_b;
  a.so_h = so_h;
  a.so_t = so_t;
  a.g = gates;
  a.sg_b = sg_b;
  a.sg_h = sg_h;
  a.sg_t = sg_t;
  a.sg_k = sg_k;
  a.out = out;
  a.sx_b = sout_b;
  a.sx_h = sout_h;
  a.sx_t = sout_t;
  a.B = B;
  a.H = H;
  a.T = T;
  a.dv = dv;
  a.act = gate_act;
  return launch_mix<false>(dtype, a, (hipStream_t)stream);
}

extern "C" int nsa_gate_mix_bwd(const void* dout, int64_t sd_b, int64_t sd_h, int64_t sd_t, const void* o_cmp,
                                const void* o_sel, const void* o_win, int64_t so_b, int64_t so_h, int64_t so_t,
                                const void* gates, int64_t sg_b, int64_t sg_h, int64_t sg_t, int64_t sg_k,
                                void* do_cmp, void* do_sel, void* do_win, float* dgates, float* delta, int B, int H,
                                int T, int dv, int gate_act, int dtype, nsa_stream_t stream) {
  using namespace nsa;
  const void* ptrs[7] = {dout, o_cmp, o_sel, o_win, do_cmp, do_sel, do_win};
  if (int rc = check_mix(dtype, B, H, T, dv, ptrs, 7)) return rc;
  if (gate_act < 0 || gate_act > 2) return set_error(NSA_ERR_INVALID, "gate_act must be 0, 1 or 2");
  const int esz = dtype == NSA_F32 ? 4 : 2;
  if ((so_t * esz) % 16 || (so_h * esz) % 16 || (sd_t * esz) % 16 || (sd_h * esz) % 16)
    return set_error(NSA_ERR_LAYOUT, "rows must be 16-byte aligned");
  MixArgs a{};
  a.o[0] = o_cmp;
  a.o[1] = o_sel;
  a.o[2] = o_win;
  a.so_b = so_b;
  a.so_h = so_h;
  a.so_t = so_t;
  a.g = gates;
  a.sg_b = sg_b;
  a.sg_h = sg_h;
  a.sg_t = sg_t;
  a.sg_k = sg_k;
  a.out = const_cast<void*>(dout);
  a.sx_b = sd_b;
  a.sx_h = sd_h;
  a.sx_t = sd_t;
  a.dO[0] = do_cmp;
  a.dO[1] = do_sel;
  a.dO[2] = do_win;
  a.dg = dgates;
  a.delta = delta;
  a.act = gate_act;
  a.B = B;
  a.H = H;
  a.T = T;
  a.dv = dv;
  return launch_mix<true>(dtype, a, (hipStream_t)stream);
}

extern "C" int nsa_gate_act_fwd(const void* gate_in, int64_t sz_b, int64_t sz_h, int64_t sz_t, int64_t sz_k,
                                float* gates, int B, int H, int T, int gate_act, int dtype, nsa_stream_t stream) {
  return nsa::launch_gate_act<false>(dtype, gate_in, gates, nullptr, nullptr, sz_b, sz_h, sz_t, sz_k, B, H, T,
                                     gate_act, (hipStream_t)stream);
}

extern "C" int nsa_gate_act_bwd(const float* gates, const float* row_dots, void* dgate_in, int64_t sz_b, int64_t sz_h,
                                int64_t sz_t, int64_t sz_k, int B, int H, int T, int gate_act, int dtype,
                                nsa_stream_t stream) {
  return nsa::launch_gate_act<true>(dtype, nullptr, const_cast<float*>(gates), row_dots, dgate_in, sz_b, sz_h, sz_t,
                                    sz_k, B, H, T, gate_act, (hipStream_t)stream);
}
