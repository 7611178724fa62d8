// Backward row statistics as a pass of their own, for the backwards whose dK/dV kernel
// runs before the dQ kernel (stored dS): per query row the record AttnArgs::rstat
//   lse2  = (M + L) * log2(e)       (+inf when L = -inf: the row saw no key)
//   delta = sum_d O[d] * dO[d]      (fp32; or the caller's precomputed delta_in)
//   gate  = row_gate[row]           (1 without a row gate)
// and row_dot (when asked) = delta (the gate's gradient, see nsa_attn_rowstats.h).
// 16 lanes per row, 16-byte pieces of O and dO, four rows per lane group.
#include "../../include/nsa_hip.h"
#include "nsa_attn.h"
#include "nsa_device.h"
#include "nsa_kernels.h"

namespace nsa {

// kStatRows rows per 16-lane group (consecutive timesteps of a head across the groups,
// so the statistics reads and writes coalesce), all their O / dO pieces requested
// before any is used
constexpr int kStatRows = 4;

template <typename T, int DV>
__global__ __launch_bounds__(256) void row_stats_kernel(AttnArgs a) {
  using S = typename Store<T>::type;
  constexpr int EPF = 16 / (int)sizeof(S);
  constexpr int NP = (DV / EPF + 15) / 16;  // 16-byte pieces per lane and row
  const int64_t nrows = (int64_t)a.B * a.H * a.Tq;
  const int l = threadIdx.x & 15;
  int64_t r[kStatRows];
  int b[kStatRows], h[kStatRows], t[kStatRows];
#pragma unroll
  for (int k = 0; k < kStatRows; ++k) {
    const int64_t row = (int64_t)blockIdx.x * (16 * kStatRows) + k * 16 + (threadIdx.x >> 4);
    r[k] = row < nrows ? row : nrows - 1;  // past the end: the last row again (not stored)
    t[k] = (int)(r[k] % a.Tq);
    const int64_t bh = r[k] / a.Tq;
    h[k] = (int)(bh % a.H);
    b[k] = (int)(bh / a.H);
  }
  float dl[kStatRows];
  {
    uint4 ov[kStatRows][NP], dv[kStatRows][NP];
#pragma unroll
    for (int k = 0; k < kStatRows; ++k) {
      const S* op = reinterpret_cast<const S*>(a.o) + b[k] * a.so_b + (int64_t)h[k] * a.so_h + (int64_t)t[k] * a.so_t;
      const S* dp = reinterpret_cast<const S*>(a.dout) + b[k] * a.sdo_b + (int64_t)h[k] * a.sdo_h +
                    (int64_t)t[k] * a.sdo_t;
#pragma unroll
      for (int j = 0; j < NP; ++j) {
        const int p = l + 16 * j;
        const bool in = p < DV / EPF;
        ov[k][j] = in ? *reinterpret_cast<const uint4*>(op + p * EPF) : make_uint4(0, 0, 0, 0);
        dv[k][j] = in ? *reinterpret_cast<const uint4*>(dp + p * EPF) : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int k = 0; k < kStatRows; ++k) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < NP; ++j) {
        const S* o = reinterpret_cast<const S*>(&ov[k][j]);
        const S* d = reinterpret_cast<const S*>(&dv[k][j]);
#pragma unroll
        for (int u = 0; u < EPF; ++u) acc = fmaf(Elem<T>::to_f32(o[u]), Elem<T>::to_f32(d[u]), acc);
      }
#pragma unroll
      for (int o = 8; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 16);
      dl[k] = acc;
    }
  }
  if (l != 0) return;
#pragma unroll
  for (int k = 0; k < kStatRows; ++k) {
    const int64_t row = (int64_t)blockIdx.x * (16 * kStatRows) + k * 16 + (threadIdx.x >> 4);
    if (row >= nrows) continue;
    const float L = a.L[b[k] * a.sl_b + (int64_t)h[k] * a.sl_h + (int64_t)t[k] * a.sl_t];
    const float M = a.M[b[k] * a.sm_b + (int64_t)h[k] * a.sm_h + (int64_t)t[k] * a.sm_t];
    const float gate = a.row_gate ? a.row_gate[r[k]] : 1.f;
    a.rstat[((int64_t)(b[k] * a.G + h[k] / a.hpg) * a.Tq + t[k]) * a.hpg + h[k] % a.hpg] =
        make_float4(L == -INFINITY ? INFINITY : (M + L) * kLog2e, dl[k], gate, 0.f);
    if (a.row_dot) a.row_dot[r[k]] = dl[k];
  }
}

// With the caller's row sums (delta_in) nothing is read per feature: one thread per row,
// rows in the record order ([B*G][Tq][hpg]) so the records are written contiguously.
__global__ __launch_bounds__(256) void row_stats_in_kernel(AttnArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)a.B * a.H * a.Tq) return;
  const int hh = (int)(i % a.hpg);
  const int64_t bt = i / a.hpg;
  const int t = (int)(bt % a.Tq);
  const int bg = (int)(bt / a.Tq);
  const int b = bg / a.G, h = (bg % a.G) * a.hpg + hh;
  const int64_t srow = ((int64_t)b * a.H + h) * a.Tq + t;
  const float L = a.L[b * a.sl_b + (int64_t)h * a.sl_h + (int64_t)t * a.sl_t];
  const float M = a.M[b * a.sm_b + (int64_t)h * a.sm_h + (int64_t)t * a.sm_t];
  a.rstat[i] = make_float4(L == -INFINITY ? INFINITY : (M + L) * kLog2e, a.delta_in[srow],
                           a.row_gate ? a.row_gate[srow] : 1.f, 0.f);
}

bool launch_row_stats(int dtype, int dv, const AttnArgs& a, hipStream_t st) {
  const int64_t nrows = (int64_t)a.B * a.H * a.Tq;
  if (a.delta_in) {
    hipLaunchKernelGGL(row_stats_in_kernel, dim3((unsigned)((nrows + 255) / 256)), dim3(256), 0, st, a);
    return true;
  }
  const dim3 grid((unsigned)((nrows + 16 * kStatRows - 1) / (16 * kStatRows)));
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

// Row dots of the gated mix (the module backward): dots[k][row] = sum_d dout . o_k for
// the three branch outputs, dout read once.  They are the gate gradient's inputs and the
// branches' delta_in, so no branch backward reads its output again.  A workgroup takes
// 16 heads x 4 timesteps: lane group g owns head h0 + g at the four timesteps, so with
// heads the contiguous axis ([B,T,H,dv] storage) the 16 groups read one contiguous run
// per timestep, and each group stores its four dots of a head as one 16-byte vector.
template <typename T, int DV>
__global__ __launch_bounds__(256) void mix_row_dots_kernel(const void* dout, const void* o0, const void* o1,
                                                           const void* o2, int64_t s_b, int64_t s_h, int64_t s_t,
                                                           float* dots, int B, int H, int Tq) {
  using S = typename Store<T>::type;
  constexpr int EPF = 16 / (int)sizeof(S);
  constexpr int NP = (DV / EPF + 15) / 16;
  const int l = threadIdx.x & 15, grp = threadIdx.x >> 4;
  // head groups fastest: the workgroups in flight together read whole timesteps' rows
  // (all heads of a timestep are one contiguous run)
  const int nhb = (H + 15) / 16;
  const int t0 = (blockIdx.x / nhb) * 4;
  const int h = (blockIdx.x % nhb) * 16 + grp;
  const int b = blockIdx.y;
  const bool hv = h < H;
  const S* src[4] = {reinterpret_cast<const S*>(dout), reinterpret_cast<const S*>(o0), reinterpret_cast<const S*>(o1),
                     reinterpret_cast<const S*>(o2)};
  int64_t off[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)  // rows past the end re-read a valid row (not stored)
    off[k] = b * s_b + (int64_t)(hv ? h : H - 1) * s_h + (int64_t)min(t0 + k, Tq - 1) * s_t;
  uint4 v[4][4][NP];
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int j = 0; j < NP; ++j) {
        const int p = l + 16 * j;
        v[x][k][j] = p < DV / EPF ? __builtin_bit_cast(uint4, __builtin_nontemporal_load(
                                        reinterpret_cast<const u32x4*>(src[x] + off[k] + p * EPF)))
                                  : make_uint4(0, 0, 0, 0);  // read once: streamed past the caches
      }
  float acc[3][4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
#pragma unroll
    for (int x = 0; x < 3; ++x) acc[x][k] = 0.f;
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const S* d = reinterpret_cast<const S*>(&v[0][k][j]);
#pragma unroll
      for (int x = 0; x < 3; ++x) {
        const S* o = reinterpret_cast<const S*>(&v[x + 1][k][j]);
#pragma unroll
        for (int u = 0; u < EPF; ++u) acc[x][k] = fmaf(Elem<T>::to_f32(o[u]), Elem<T>::to_f32(d[u]), acc[x][k]);
      }
    }
#pragma unroll
    for (int x = 0; x < 3; ++x)
#pragma unroll
      for (int o = 8; o >= 1; o >>= 1) acc[x][k] += __shfl_xor(acc[x][k], o, 16);
  }
  if (l != 0 || !hv) return;
  const int64_t plane = (int64_t)B * H * Tq;
#pragma unroll
  for (int x = 0; x < 3; ++x) {
    float* dp = dots + x * plane + ((int64_t)b * H + h) * Tq + t0;
    if (t0 + 3 < Tq && (reinterpret_cast<uintptr_t>(dp) & 15) == 0) {
      *reinterpret_cast<float4*>(dp) = make_float4(acc[x][0], acc[x][1], acc[x][2], acc[x][3]);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (t0 + k < Tq) dp[k] = acc[x][k];
    }
  }
}

}  // namespace nsa

extern "C" int nsa_mix_row_dots(const void* dout, const void* o_cmp, const void* o_sel, const void* o_win,
                                int64_t so_b, int64_t so_h, int64_t so_t, float* dots, int B, int H, int T, int dv,
                                int dtype, nsa_stream_t stream) {
  using namespace nsa;
  if (dtype != NSA_F32 && dtype != NSA_BF16) return set_error(NSA_ERR_INVALID, "dtype not supported");
  if (B < 0 || H < 0 || T < 0) return set_error(NSA_ERR_INVALID, "bad shape");
  const int64_t nrows = (int64_t)B * H * T;
  if (nrows == 0) return NSA_OK;
  if (!dout || !o_cmp || !o_sel || !o_win || !dots) return set_error(NSA_ERR_INVALID, "null pointer");
  const int esz = dtype == NSA_F32 ? 4 : 2;
  const void* ptrs[4] = {dout, o_cmp, o_sel, o_win};
  for (const void* p : ptrs)
    if ((uintptr_t)p % 16) return set_error(NSA_ERR_LAYOUT, "rows must be 16-byte aligned");
  if ((so_t * esz) % 16 || (so_h * esz) % 16 || (so_b * esz) % 16)
    return set_error(NSA_ERR_LAYOUT, "rows must be 16-byte aligned");
  const dim3 grid((unsigned)(((T + 3) / 4) * ((H + 15) / 16)), (unsigned)B);
  hipStream_t st = (hipStream_t)stream;
#define NSA_DOTS(DVV)                                                                                             \
  if (dv == DVV) {                                                                                                \
    if (dtype == NSA_BF16)                                                                                        \
      hipLaunchKernelGGL((mix_row_dots_kernel<bf16, DVV>), grid, dim3(256), 0, st, dout, o_cmp, o_sel, o_win, so_b, \
                         so_h, so_t, dots, B, H, T);                                                              \
    else                                                                                                          \
      hipLaunchKernelGGL((mix_row_dots_kernel<float, DVV>), grid, dim3(256), 0, st, dout, o_cmp, o_sel, o_win,    \
                         so_b, so_h, so_t, dots, B, H, T);                                                        \
    hipError_t e = hipGetLastError();                                                                             \
    return e == hipSuccess ? NSA_OK : set_error(NSA_ERR_HIP, hipGetErrorString(e));                              \
  }
  NSA_DOTS(32)
  NSA_DOTS(64)
  NSA_DOTS(128)
#undef NSA_DOTS
  return set_error(NSA_ERR_UNSUPPORTED, "head_dim_v must be 32, 64 or 128");
}
