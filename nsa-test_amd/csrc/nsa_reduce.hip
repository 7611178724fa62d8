// dK/dV partial reduction and the dtype dispatch of the attention kernels.
//
// Compression and selection split a key tile's queries over several work items;
// each item wrote fp32 partials [keys][DK + DV].  One workgroup per key tile
// sums them in item order (fixed, so the result is reproducible) and accumulates
// into the caller's dK / dV with their strides.
#include "nsa_attn.h"
#include "nsa_attn_bwd_dkdv.h"
#include "nsa_device.h"
#include "nsa_kernels.h"

namespace nsa {

constexpr int kReduceSplit = 10;

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
__global__ __launch_bounds__(256) void partial_reduce_kernel(AttnArgs a, int DK, int DV, int br) {
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
  if (count == 0 || key0 >= key_hi) return;
  const float* base = a.partial + (int64_t)bg * a.items_per_bg * keys * width;
  // blockIdx.z splits the tile's keys x width elements (in groups of four: DK and DV are
  // multiples of four, so a group never straddles dK / dV) over kReduceSplit workgroups
  const int n4 = keys * width / 4;
  const int per = (n4 + kReduceSplit - 1) / kReduceSplit;
  const int e_end = min(n4, (int)(blockIdx.z + 1) * per);
  for (int e4 = blockIdx.z * per + threadIdx.x; e4 < e_end; e4 += 256) {
    const int e = 4 * e4;
    const int kl = e / width, col = e % width;
    const int key = key0 + kl;
    if (key >= key_hi) continue;
    float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k = 0; k < count; ++k) {
      const float4 v = *reinterpret_cast<const float4*>(base + (int64_t)(first + k * step) * keys * width + e);
      sum.x += v.x;
      sum.y += v.y;
      sum.z += v.z;
      sum.w += v.w;
    }
    const float sv[4] = {sum.x, sum.y, sum.z, sum.w};
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
    if (sd == 1 && (reinterpret_cast<uintptr_t>(p) % (4 * sizeof(S))) == 0) {  // one vector read-modify-write
      if constexpr (sizeof(S) == 2) {
        uint2 w = *reinterpret_cast<const uint2*>(p);
        const float x0 = bf16_bits_to_f32((uint16_t)(w.x & 0xffffu)) + sv[0];
        const float x1 = bf16_bits_to_f32((uint16_t)(w.x >> 16)) + sv[1];
        const float x2 = bf16_bits_to_f32((uint16_t)(w.y & 0xffffu)) + sv[2];
        const float x3 = bf16_bits_to_f32((uint16_t)(w.y >> 16)) + sv[3];
        w.x = (uint32_t)f32_to_bf16_bits(x0) | ((uint32_t)f32_to_bf16_bits(x1) << 16);
        w.y = (uint32_t)f32_to_bf16_bits(x2) | ((uint32_t)f32_to_bf16_bits(x3) << 16);
        *reinterpret_cast<uint2*>(p) = w;
      } else {
        float4 w = *reinterpret_cast<const float4*>(p);
        w.x += sv[0];
        w.y += sv[1];
        w.z += sv[2];
        w.w += sv[3];
        *reinterpret_cast<float4*>(p) = w;
      }
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) p[u * sd] = Elem<T>::from_f32(Elem<T>::to_f32(p[u * sd]) + sv[u]);
    }
  }
}

void launch_partial_reduce(int dtype, int dk, int dv, int br, const AttnArgs& a, hipStream_t st) {
  int tiles;
  if (br != kSelection) tiles = (a.Tkv + dkdv_keys(br) - 1) / dkdv_keys(br);
  else tiles = a.nblk * ((a.lprime + 63) / 64);
  if (tiles <= 0) return;
  dim3 grid(tiles, a.B * a.G, kReduceSplit);
  if (dtype == kF32)
    hipLaunchKernelGGL(partial_reduce_kernel<float>, grid, dim3(256), 0, st, a, dk, dv, br);
  else
    hipLaunchKernelGGL(partial_reduce_kernel<bf16>, grid, dim3(256), 0, st, a, dk, dv, br);
}

}  // namespace nsa
