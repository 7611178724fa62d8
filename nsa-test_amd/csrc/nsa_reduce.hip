// dK/dV partial reduction and the dtype dispatch of the attention kernels.
//
// Compression and selection split a key tile's queries over several work items;
// each item wrote fp32 partials [64 keys][DK + DV].  One workgroup per key tile
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
  if (br != kSelection) {
    const int nseg = dkdv_nseg(br, a.Tq, a.window);
    key0 = blockIdx.x * 64;
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
  const float* base = a.partial + (int64_t)bg * a.items_per_bg * 64 * width;
  // blockIdx.z splits the tile's 64 x width elements over kReduceSplit workgroups
  const int per = (64 * width + kReduceSplit - 1) / kReduceSplit;
  const int e_end = min(64 * width, (int)(blockIdx.z + 1) * per);
  for (int e = blockIdx.z * per + threadIdx.x; e < e_end; e += 256) {
    const int kl = e / width, col = e % width;
    const int key = key0 + kl;
    if (key >= key_hi) continue;
    float sum = 0.f;
    for (int k = 0; k < count; ++k) sum += base[(int64_t)(first + k * step) * 64 * width + e];
    if (col < DK) {
      S* p = reinterpret_cast<S*>(a.dk) + b * a.sdk_b + grp * a.sdk_g + (int64_t)key * a.sdk_t + (int64_t)col * a.sdk_d;
      *p = Elem<T>::from_f32(Elem<T>::to_f32(*p) + sum);
    } else {
      S* p = reinterpret_cast<S*>(a.dv) + b * a.sdv_b + grp * a.sdv_g + (int64_t)key * a.sdv_t +
             (int64_t)(col - DK) * a.sdv_d;
      *p = Elem<T>::from_f32(Elem<T>::to_f32(*p) + sum);
    }
  }
}

void launch_partial_reduce(int dtype, int dk, int dv, int br, const AttnArgs& a, hipStream_t st) {
  int tiles;
  if (br != kSelection) tiles = (a.Tkv + 63) / 64;
  else tiles = a.nblk * ((a.lprime + 63) / 64);
  if (tiles <= 0) return;
  dim3 grid(tiles, a.B * a.G, kReduceSplit);
  if (dtype == kF32)
    hipLaunchKernelGGL(partial_reduce_kernel<float>, grid, dim3(256), 0, st, a, dk, dv, br);
  else
    hipLaunchKernelGGL(partial_reduce_kernel<bf16>, grid, dim3(256), 0, st, a, dk, dv, br);
}

}  // namespace nsa
