// Backward row statistics as a pass of their own, for the branches whose dK/dV kernel
// runs before the dQ kernel (the selection backward with stored dS): per query row
//   lse2  = (M + L) * log2(e)       (+inf when L = -inf: the row saw no key)
//   delta = sum_d O[d] * dO[d]      (fp32; or the caller's precomputed delta_in)
//   row_dot (when asked)  = delta   (the gate's gradient, see nsa_attn_rowstats.h)
// 16 lanes per row, 16-byte pieces of O and dO.
#include "nsa_attn.h"
#include "nsa_device.h"
#include "nsa_kernels.h"

namespace nsa {

template <typename T, int DV>
__global__ __launch_bounds__(256) void row_stats_kernel(AttnArgs a) {
  using S = typename Store<T>::type;
  constexpr int EPF = 16 / (int)sizeof(S);
  constexpr int NP = DV / EPF;  // 16-byte pieces per row
  const int64_t nrows = (int64_t)a.B * a.H * a.Tq;
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int l = threadIdx.x & 15;
  const bool ok = row < nrows;
  const int64_t r = ok ? row : 0;
  const int t = (int)(r % a.Tq);
  const int64_t bh = r / a.Tq;
  const int h = (int)(bh % a.H), b = (int)(bh / a.H);
  float dl = 0.f;
  if (a.delta_in) {
    dl = a.delta_in[r];
  } else {
    const S* op = reinterpret_cast<const S*>(a.o) + b * a.so_b + (int64_t)h * a.so_h + (int64_t)t * a.so_t;
    const S* dp = reinterpret_cast<const S*>(a.dout) + b * a.sdo_b + (int64_t)h * a.sdo_h + (int64_t)t * a.sdo_t;
    float acc = 0.f;
#pragma unroll
    for (int p = l; p < NP; p += 16) {
      const uint4 ov = *reinterpret_cast<const uint4*>(op + p * EPF);
      const uint4 dv = *reinterpret_cast<const uint4*>(dp + p * EPF);
      const S* o = reinterpret_cast<const S*>(&ov);
      const S* d = reinterpret_cast<const S*>(&dv);
#pragma unroll
      for (int u = 0; u < EPF; ++u) acc = fmaf(Elem<T>::to_f32(o[u]), Elem<T>::to_f32(d[u]), acc);
    }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 16);
    dl = acc;
  }
  if (!ok || l != 0) return;
  const float L = a.L[b * a.sl_b + (int64_t)h * a.sl_h + (int64_t)t * a.sl_t];
  const float M = a.M[b * a.sm_b + (int64_t)h * a.sm_h + (int64_t)t * a.sm_t];
  const_cast<float*>(a.lse2)[r] = L == -INFINITY ? INFINITY : (M + L) * kLog2e;
  const_cast<float*>(a.delta)[r] = dl;
  if (a.row_dot) a.row_dot[r] = dl;
}

bool launch_row_stats(int dtype, int dv, const AttnArgs& a, hipStream_t st) {
  const int64_t nrows = (int64_t)a.B * a.H * a.Tq;
  const dim3 grid((unsigned)((nrows + 15) / 16));
#define NSA_ROWSTATS(DVV)                                                                             \
  if (dv == DVV) {                                                                                    \
    if (dtype == kBF16) hipLaunchKernelGGL((row_stats_kernel<bf16, DVV>), grid, dim3(256), 0, st, a); \
    else hipLaunchKernelGGL((row_stats_kernel<float, DVV>), grid, dim3(256), 0, st, a);               \
    return true;                                                                                      \
  }
  NSA_ROWSTATS(32)
  NSA_ROWSTATS(64)
  NSA_ROWSTATS(128)
#undef NSA_ROWSTATS
  return false;
}

}  // namespace nsa
