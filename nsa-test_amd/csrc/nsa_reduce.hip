// dK/dV partial reduction and the dtype dispatch of the attention kernels.
//
// Compression and selection split a key tile's queries over several work items;
// each item wrote partials [keys][DK + DV] in the element type (fp32 / bf16), summed here
// in fp32.  One workgroup per key tile
// sums them in item order (fixed, so the result is reproducible) and accumulates
// into the caller's dK / dV with their strides (or, in overwrite mode, stores the sum:
// a tile without items then stores zeros).
#include <algorithm>
#include "nsa_attn.h"
#include "nsa_attn_bwd_dkdv.h"
#include "nsa_device.h"
#include "nsa_kernels.h"

namespace nsa {

constexpr int kReduceSplit = 20;

bool dispatch_attn_fwd_f32(int, int, int, const AttnArgs&, hipStream_t);
bool dispatch_attn_fwd_bf16(int, int, int, const AttnArgs&, hipStream_t);
bool dispatch_attn_bwd_dq_f32(int, int, int, const AttnArgs&, hipStream_t);
bool dispatch_attn_bwd_dq_bf16(int, int, int, const AttnArgs&, hipStream_t);
bool dispatch_attn_bwd_dkdv_f32(int, int, int, const AttnArgs&, hipStream_t);
bool dispatch_attn_bwd_dkdv_bf16(int, int, int, const AttnArgs&, hipStream_t);

bool dispatch_attn_fwd(int dtype, int dk, int dv, int br, const AttnArgs& a, hipStream_t st) {
  return dtype == kF32 ? dispatch_attn_fwd_f32(dk, dv, br, a, st) : dispatch_attn_fwd_bf16(dk, dv, br, a, st);
}
bool dispatch_attn_bwd_dq(int dtype, int dk, int dv, int br, const AttnArgs& a, hipStream_t st) {
  return dtype == kF32 ? dispatch_attn_bwd_dq_f32(dk, dv, br, a, st) : dispatch_attn_bwd_dq_bf16(dk, dv, br, a, st);
}
bool dispatch_attn_bwd_dkdv(int dtype, int dk, int dv, int br, const AttnArgs& a, hipStream_t st) {
  return dtype == kF32 ? dispatch_attn_bwd_dkdv_f32(dk, dv, br, a, st)
                       : dispatch_attn_bwd_dkdv_bf16(dk, dv, br, a, st);
}

template <typename T>
__global__ __launch_bounds__(256) void partial_reduce_kernel(AttnArgs a, int DK, int DV, int br, int split) {
  using S = typename Store<T>::type;
  const int bg = blockIdx.y;
  const int b = bg / a.G, grp = bg % a.G;
  const int width = DK + DV;
  int key0, key_hi, first, count, step;
  const int keys = dkdv_keys(br);  // keys of one item's partial
  if (br != kSelection) {
    const int nseg = dkdv_nseg(br, a.Tq, a.window, a.seg);
    key0 = blockIdx.x * keys;
    key_hi = a.Tkv;
    first = blockIdx.x * nseg;
    count = nseg;
    step = 1;
  } else {
    const int nsubblk = (a.lprime + 63) / 64;
    const int j = blockIdx.x / nsubblk, sub = blockIdx.x % nsubblk;
    const int* so = a.seg_off + (int64_t)bg * (a.nblk + 1);
    key0 = j * a.lprime + sub * 64;
    key_hi = min(j * a.lprime + a.lprime, a.Tkv);
    first = so[j] * nsubblk + sub;
    count = so[j + 1] - so[j];
    step = nsubblk;
  }
  if ((count == 0 && !a.dkdv_ow) || key0 >= key_hi) return;
  const S* base = reinterpret_cast<const S*>(a.partial) + (int64_t)bg * a.items_per_bg * keys * width;
  const int64_t istride = (int64_t)step * keys * width;  // elements between consecutive items
  // each thread sums a group of NE consecutive elements (16 bytes of every partial: DK
  // and DV are multiples of NE, so a group never straddles dK / dV); blockIdx.z splits
  // the tile's keys x width elements over `split` workgroups
  constexpr int NE = 16 / sizeof(S);
  const int ng = keys * width / NE;
  const int per = (ng + split - 1) / split;
  const int g_end = min(ng, (int)(blockIdx.z + 1) * per);
  for (int gi = blockIdx.z * per + threadIdx.x; gi < g_end; gi += 256) {
    const int e = NE * gi;
    const int kl = e / width, col = e % width;
    const int key = key0 + kl;
    if (key >= key_hi) continue;
    S* p;
    int64_t sd;
    if (col < DK) {
      p = reinterpret_cast<S*>(a.dk) + b * a.sdk_b + grp * a.sdk_g + (int64_t)key * a.sdk_t + (int64_t)col * a.sdk_d;
      sd = a.sdk_d;
    } else {
      p = reinterpret_cast<S*>(a.dv) + b * a.sdv_b + grp * a.sdv_g + (int64_t)key * a.sdv_t +
          (int64_t)(col - DK) * a.sdv_d;
      sd = a.sdv_d;
    }
    const bool vec = sd == 1 && (reinterpret_cast<uintptr_t>(p) % 16) == 0;
    const bool ow = a.dkdv_ow;
    // the destination's current values are requested first (independent of the sum)
    uint4 old = make_uint4(0u, 0u, 0u, 0u);
    if (vec && !ow) old = *reinterpret_cast<const uint4*>(p);
    // the items' partials in item order (fixed: reproducible), eight (then four) loads in
    // flight; each partial is read once, so the loads stream past the caches
    const S* src = base + (int64_t)first * keys * width + e;
    auto ld = [&](int k) -> uint4 {
      return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + k * istride)));
    };
    float sum[NE];
#pragma unroll
    for (int u = 0; u < NE; ++u) sum[u] = 0.f;
    auto add = [&](const uint4& v) {
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
      if constexpr (NE == 8) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          sum[2 * u] += __uint_as_float(w[u] << 16);
          sum[2 * u + 1] += __uint_as_float(w[u] & 0xffff0000u);
        }
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) sum[u] += __uint_as_float(w[u]);
      }
    };
    int k = 0;
    for (; k + 8 <= count; k += 8) {
      uint4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = ld(k + u);
#pragma unroll
      for (int u = 0; u < 8; ++u) add(v[u]);
    }
    for (; k + 4 <= count; k += 4) {
      uint4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = ld(k + u);
#pragma unroll
      for (int u = 0; u < 4; ++u) add(v[u]);
    }
    for (; k < count; ++k) add(ld(k));
    if (vec) {  // one vector store (read-modify-write when accumulating)
      if (!ow) {
        const uint32_t w[4] = {old.x, old.y, old.z, old.w};
        if constexpr (NE == 8) {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            sum[2 * u] += __uint_as_float(w[u] << 16);
            sum[2 * u + 1] += __uint_as_float(w[u] & 0xffff0000u);
          }
        } else {
#pragma unroll
          for (int u = 0; u < 4; ++u) sum[u] += __uint_as_float(w[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < NE; u += 4) store4<T>(p + u, f32x4{sum[u], sum[u + 1], sum[u + 2], sum[u + 3]});
    } else if (ow) {
#pragma unroll
      for (int u = 0; u < NE; ++u) p[u * sd] = Elem<T>::from_f32(sum[u]);
    } else {
#pragma unroll
      for (int u = 0; u < NE; ++u) p[u * sd] = Elem<T>::from_f32(Elem<T>::to_f32(p[u * sd]) + sum[u]);
    }
  }
}

// Overwrite mode with no query rows: dK / dV [B, G, Tkv, dk | dv] (any strides) set to 0.
template <typename T>
__global__ __launch_bounds__(256) void zero_dkdv_kernel(AttnArgs a, int DK, int DV) {
  using S = typename Store<T>::type;
  const int bg = blockIdx.y, b = bg / a.G, grp = bg % a.G;
  const int width = DK + DV;
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (int64_t)a.Tkv * width) return;
  const int key = (int)(e / width), col = (int)(e % width);
  S* p = col < DK ? reinterpret_cast<S*>(a.dk) + b * a.sdk_b + grp * a.sdk_g + (int64_t)key * a.sdk_t +
                        (int64_t)col * a.sdk_d
                  : reinterpret_cast<S*>(a.dv) + b * a.sdv_b + grp * a.sdv_g + (int64_t)key * a.sdv_t +
                        (int64_t)(col - DK) * a.sdv_d;
  *p = Elem<T>::from_f32(0.f);
}

void launch_zero_dkdv(int dtype, int dk, int dv, const AttnArgs& a, hipStream_t st) {
  const int64_t n = (int64_t)a.Tkv * (dk + dv);
  if (n <= 0 || a.B * a.G <= 0) return;
  dim3 grid((unsigned)((n + 255) / 256), a.B * a.G);
  if (dtype == kF32) hipLaunchKernelGGL(zero_dkdv_kernel<float>, grid, dim3(256), 0, st, a, dk, dv);
  else hipLaunchKernelGGL(zero_dkdv_kernel<bf16>, grid, dim3(256), 0, st, a, dk, dv);
}

void launch_partial_reduce(int dtype, int dk, int dv, int br, const AttnArgs& a, hipStream_t st) {
  int tiles;
  if (br != kSelection) tiles = (a.Tkv + dkdv_keys(br) - 1) / dkdv_keys(br);
  else tiles = a.nblk * ((a.lprime + 63) / 64);
  if (tiles <= 0) return;
  // at least ~2048 workgroups (few key tiles: compression), each with one or more float4
  // groups per thread
  const int n4 = dkdv_keys(br) * (dk + dv) / 4;
  const int64_t tb = (int64_t)tiles * a.B * a.G;
  int split = (int)std::min<int64_t>(std::max<int64_t>(kReduceSplit, (2048 + tb - 1) / tb), (n4 + 255) / 256);
  split = std::max(split, 1);
  dim3 grid(tiles, a.B * a.G, split);
  if (dtype == kF32)
    hipLaunchKernelGGL(partial_reduce_kernel<float>, grid, dim3(256), 0, st, a, dk, dv, br, split);
  else
    hipLaunchKernelGGL(partial_reduce_kernel<bf16>, grid, dim3(256), 0, st, a, dk, dv, br, split);
}

}  // namespace nsa
