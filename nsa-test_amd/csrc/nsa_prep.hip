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

// One repack of a fragment-layout copy: its source, width and the outputs it fills.
// Feature-contiguous source (tr = 0): unit feature stride, 16-byte aligned rows, s_x the
// row stride.  Time-contiguous source (tr = 1: K in the reference's [B,G,dk,T] layout):
// unit row stride, 16-byte aligned feature runs, s_x the feature stride.
template <typename S>
struct RepackJob {
  const S* src;
  int64_t s_b, s_g, s_x;
  int C;
  int tr;
  S* rowf;
  S* colf;
};

// LDS tile of one 64 x 64 repack step: 64 lines of 64 + EPF elements (16-byte aligned
// lines; strided reads spread over the banks)
template <typename S>
constexpr int kRepackPitch = 64 + 16 / (int)sizeof(S);

// Fragment layouts from a feature-contiguous source: the 64 x 64 tile is read as 16-byte
// pieces into LDS row-major (rows >= R zero), then every output 16-byte piece is written
// in output order -- a rowfrag piece is EPF consecutive features of one row (one LDS
// read), a colfrag piece gathers EPF rows of one feature (the C-permuted key order of
// CFrag for bf16).
template <typename S>
__device__ __forceinline__ void repack_rows_tile(const RepackJob<S>& j, S* tile, int G, int R, int Rp, int r0,
                                                 int c0) {
  using T = typename std::conditional<sizeof(S) == 2, bf16, float>::type;
  constexpr int EPF = 16 / sizeof(S);
  constexpr int KC = Elem<T>::kKChunk;
  constexpr int CK = CFrag<T>::kKeys;
  constexpr int P = kRepackPitch<S>;
  const int C = j.C;
  S* __restrict__ rowf = j.rowf;
  S* __restrict__ colf = j.colf;
  const int bg = blockIdx.z;
  const int b = bg / G, g = bg % G;
  const S* base = j.src + b * j.s_b + g * j.s_g;
  const int64_t s_r = j.s_x;
  const int tid = threadIdx.x;
  constexpr int PPR = 64 / EPF;  // 16-byte pieces per tile row
  for (int q = tid; q < 64 * PPR; q += 256) {
    const int rr = q / PPR, pc = (q % PPR) * EPF;
    const int r = r0 + rr, c = c0 + pc;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (r < R && c < C) v = *reinterpret_cast<const uint4*>(base + (int64_t)r * s_r + c);
    *reinterpret_cast<uint4*>(&tile[rr * P + pc]) = v;
  }
  __syncthreads();
  const int64_t obase = (int64_t)bg * Rp * C;
  if (rowf) {  // fragments (row16, kc) of the tile, 64 pieces each
    constexpr int NKCT = 64 / KC;
    for (int q = tid; q < 4 * NKCT * 64; q += 256) {
      const int fr = q >> 6, ln = q & 63;
      const int rr = (fr / NKCT) * 16 + (ln & 15);
      const int cc = (fr % NKCT) * KC + (ln >> 4) * EPF;
      const int r = r0 + rr, c = c0 + cc;
      if (r < Rp && c < C)
        *reinterpret_cast<uint4*>(rowf + obase + rowfrag_off<T>(r, c, C)) =
            *reinterpret_cast<const uint4*>(&tile[rr * P + cc]);
    }
  }
  if (colf) {  // fragments (key chunk, feature group) of the tile
    for (int q = tid; q < (64 / CK) * 4 * 64; q += 256) {
      const int fr = q >> 6, ln = q & 63;
      const int ch = fr >> 2, fg = fr & 3;
      const int gl = ln >> 4, f = ln & 15;
      const int cc = fg * 16 + f;
      const int c = c0 + cc;
      S e[EPF];
#pragma unroll
      for (int p = 0; p < EPF; ++p) {
        const int k = CK == 32 ? (p < 4 ? 4 * gl + p : 12 + 4 * gl + p) : 4 * gl + p;  // key within the chunk
        e[p] = tile[(ch * CK + k) * P + cc];
      }
      const int r = r0 + ch * CK;  // the chunk's first key; the piece's keys share its offset
      if (r < Rp && c < C) {
        uint4 v;
        __builtin_memcpy(&v, e, 16);
        *reinterpret_cast<uint4*>(colf + obase + colfrag_off<T>(r + 4 * gl, c, C)) = v;
      }
    }
  }
}

// The fragment layouts from a time-contiguous source, vectorised: each thread reads
// 16-byte runs along time into an LDS tile held feature-major, and writes whole 16-byte
// fragment pieces (rowfrag: EPF consecutive features of one row; colfrag: the EPF rows of
// one C-permuted slot group of one feature).  Rows R..Rp-1 are zero.
template <typename S>
__device__ __forceinline__ void repack_time_tile(const RepackJob<S>& j, S* tile, int G, int R, int Rp, int r0,
                                                 int c0) {
  using T = typename std::conditional<sizeof(S) == 2, bf16, float>::type;
  constexpr int EPF = 16 / (int)sizeof(S);
  constexpr int CK = CFrag<T>::kKeys;
  constexpr int P = kRepackPitch<S>;
  const int C = j.C;
  S* __restrict__ rowf = j.rowf;
  S* __restrict__ colf = j.colf;
  const int bg = blockIdx.z;
  const int b = bg / G, g = bg % G;
  const S* base = j.src + b * j.s_b + g * j.s_g;
  const int64_t s_c = j.s_x;
  const int tid = threadIdx.x;
  constexpr int NP = 64 * 64 / EPF / 256;  // pieces per thread
#pragma unroll
  for (int k = 0; k < NP; ++k) {
    const int i = tid + 256 * k;
    const int cc = i / (64 / EPF), rp = (i % (64 / EPF)) * EPF;
    const int c = c0 + cc, r = r0 + rp;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (c < C) {
      const S* p = base + (int64_t)c * s_c + r;
      if (r + EPF <= R) {
        v = *reinterpret_cast<const uint4*>(p);
      } else {
        S e[EPF];
#pragma unroll
        for (int u = 0; u < EPF; ++u) e[u] = r + u < R ? p[u] : S(0);
        v = *reinterpret_cast<const uint4*>(e);
      }
    }
    *reinterpret_cast<uint4*>(&tile[cc * P + rp]) = v;
  }
  __syncthreads();
  const int64_t obase = (int64_t)bg * Rp * C;
  if (rowf) {
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const int i = tid + 256 * k;
      const int rr = i / (64 / EPF), cp = (i % (64 / EPF)) * EPF;
      const int r = r0 + rr, c = c0 + cp;
      if (r < Rp && c < C) {
        S e[EPF];
#pragma unroll
        for (int u = 0; u < EPF; ++u) e[u] = tile[(cp + u) * P + rr];
        *reinterpret_cast<uint4*>(rowf + obase + rowfrag_off<T>(r, c, C)) = *reinterpret_cast<const uint4*>(e);
      }
    }
  }
  if (colf) {
    // piece (key chunk, feature, slot group q): the rows at slots EPF q .. EPF q + EPF - 1
    // of the chunk's order (bf16: keys 4q..4q+3 and 16+4q..16+4q+3; fp32: 4q..4q+3)
    constexpr int NQ = CK / EPF;
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const int i = tid + 256 * k;
      const int q = i % NQ, cc = (i / NQ) % 64, ch = i / NQ / 64;
      const int rk = ch * CK + 4 * q;  // tile row of the piece's first key
      const int r = r0 + rk, c = c0 + cc;
      if (r < Rp && c < C) {
        S e[EPF];
#pragma unroll
        for (int u = 0; u < 4; ++u) e[u] = tile[cc * P + rk + u];
        if constexpr (EPF == 8) {
#pragma unroll
          for (int u = 0; u < 4; ++u) e[4 + u] = tile[cc * P + rk + 16 + u];
        }
        *reinterpret_cast<uint4*>(colf + obase + colfrag_off<T>(r, c, C)) = *reinterpret_cast<const uint4*>(e);
      }
    }
  }
}

// Fragment layouts of up to two sources in one launch (K and V of one call): column
// tiles [0, ytiles0) of blockIdx.y are job 0's, the rest job 1's; each job's source is
// feature- or time-contiguous (its tr flag, uniform over the workgroup).
template <typename S>
__global__ __launch_bounds__(256) void repack_frag_kernel(RepackJob<S> j0, RepackJob<S> j1, int ytiles0, int G,
                                                          int R, int Rp) {
  __shared__ __attribute__((aligned(16))) S tile[64 * kRepackPitch<S>];
  const bool second = (int)blockIdx.y >= ytiles0;
  const RepackJob<S>& j = second ? j1 : j0;
  const int r0 = blockIdx.x * 64, c0 = (second ? blockIdx.y - ytiles0 : blockIdx.y) * 64;
  if (j.tr)
    repack_time_tile(j, tile, G, R, Rp, r0, c0);
  else
    repack_rows_tile(j, tile, G, R, Rp, r0, c0);
}

static bool repack_tr_ok(int dtype, const void* src, int64_t s_b, int64_t s_g, int64_t s_r, int64_t s_c, int B,
                         int G, int C) {
  const int epf = dtype == kF32 ? 4 : 8;
  return s_r == 1 && C % epf == 0 && ((uintptr_t)src) % 16 == 0 && (B == 1 || s_b % epf == 0) &&
         (G == 1 || s_g % epf == 0) && s_c % epf == 0;
}

static bool repack_vec_ok(int dtype, const void* src, int64_t s_b, int64_t s_g, int64_t s_r, int64_t s_c, int B,
                          int G, int R, int C) {
  const int epf = dtype == kF32 ? 4 : 8;
  return s_c == 1 && C % epf == 0 && ((uintptr_t)src) % 16 == 0 && (B == 1 || s_b % epf == 0) &&
         (G == 1 || s_g % epf == 0) && (R <= 1 || s_r % epf == 0);
}

void launch_repack(int dtype, const void* src, int64_t s_b, int64_t s_g, int64_t s_r, int64_t s_c, int B, int G,
                   int R, int C, int Rp, void* rowm, void* colm, void* rowf, void* colf, hipStream_t st) {
  if (!rowm && !colm && !rowf && !colf) return;
  dim3 grid((Rp + 63) / 64, (C + 63) / 64, B * G);
  if (!rowm && !colm) {
    const bool vec = repack_vec_ok(dtype, src, s_b, s_g, s_r, s_c, B, G, R, C);
    if (vec || repack_tr_ok(dtype, src, s_b, s_g, s_r, s_c, B, G, C)) {
      const int64_t sx = vec ? s_r : s_c;
      if (dtype == kF32) {
        const RepackJob<float> j{(const float*)src, s_b, s_g, sx, C, vec ? 0 : 1, (float*)rowf, (float*)colf};
        hipLaunchKernelGGL(repack_frag_kernel<float>, grid, dim3(256), 0, st, j, j, (int)grid.y, G, R, Rp);
      } else {
        const RepackJob<uint16_t> j{(const uint16_t*)src, s_b, s_g, sx, C, vec ? 0 : 1, (uint16_t*)rowf,
                                    (uint16_t*)colf};
        hipLaunchKernelGGL(repack_frag_kernel<uint16_t>, grid, dim3(256), 0, st, j, j, (int)grid.y, G, R, Rp);
      }
      return;
    }
  }
  if (dtype == kF32) {
    hipLaunchKernelGGL(repack_kernel<float>, grid, dim3(256), 0, st, (const float*)src, s_b, s_g, s_r, s_c, G, R, C,
                       Rp, (float*)rowm, (float*)colm, (float*)rowf, (float*)colf);
  } else {
    hipLaunchKernelGGL(repack_kernel<uint16_t>, grid, dim3(256), 0, st, (const uint16_t*)src, s_b, s_g, s_r, s_c, G,
                       R, C, Rp, (uint16_t*)rowm, (uint16_t*)colm, (uint16_t*)rowf, (uint16_t*)colf);
  }
}

// How the fragment-only kernel reads a source: 0 feature-contiguous, 1 time-contiguous,
// -1 neither (the general kernel takes it)
static int repack_frag_mode(int dtype, const void* src, const int64_t* st, int B, int G, int R, int C) {
  if (repack_vec_ok(dtype, src, st[0], st[1], st[2], st[3], B, G, R, C)) return 0;
  if (repack_tr_ok(dtype, src, st[0], st[1], st[2], st[3], B, G, C)) return 1;
  return -1;
}

// The fragment copies of K and V for one call in one launch when both sources suit the
// fragment-only kernel (column tiles of K first, then V's; each source feature- or
// time-contiguous), else one launch each.
void launch_repack_kv(int dtype, const void* k, const int64_t* sk, int dk, void* krf, void* kcf, const void* v,
                      const int64_t* sv, int dv, void* vrf, void* vcf, int B, int G, int R, int Rp, hipStream_t st) {
  const bool kany = krf || kcf, vany = vrf || vcf;
  const int mk = kany && vany ? repack_frag_mode(dtype, k, sk, B, G, R, dk) : -1;
  const int mv = kany && vany ? repack_frag_mode(dtype, v, sv, B, G, R, dv) : -1;
  if (mk >= 0 && mv >= 0) {
    const int yk = (dk + 63) / 64;
    const dim3 grid((Rp + 63) / 64, yk + (dv + 63) / 64, B * G);
    const int64_t xk = mk ? sk[3] : sk[2], xv = mv ? sv[3] : sv[2];
    if (dtype == kF32) {
      const RepackJob<float> jk{(const float*)k, sk[0], sk[1], xk, dk, mk, (float*)krf, (float*)kcf};
      const RepackJob<float> jv{(const float*)v, sv[0], sv[1], xv, dv, mv, (float*)vrf, (float*)vcf};
      hipLaunchKernelGGL(repack_frag_kernel<float>, grid, dim3(256), 0, st, jk, jv, yk, G, R, Rp);
    } else {
      const RepackJob<uint16_t> jk{(const uint16_t*)k, sk[0], sk[1], xk, dk, mk, (uint16_t*)krf, (uint16_t*)kcf};
      const RepackJob<uint16_t> jv{(const uint16_t*)v, sv[0], sv[1], xv, dv, mv, (uint16_t*)vrf, (uint16_t*)vcf};
      hipLaunchKernelGGL(repack_frag_kernel<uint16_t>, grid, dim3(256), 0, st, jk, jv, yk, G, R, Rp);
    }
    return;
  }
  launch_repack(dtype, k, sk[0], sk[1], sk[2], sk[3], B, G, R, dk, Rp, nullptr, nullptr, krf, kcf, st);
  launch_repack(dtype, v, sv[0], sv[1], sv[2], sv[3], B, G, R, dv, Rp, nullptr, nullptr, vrf, vcf, st);
}

}  // namespace nsa
