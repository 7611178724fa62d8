// Device-side building blocks shared by every NSA kernel on gfx950 (CDNA4).
//
// Matrix products run on 16x16 MFMA tiles:
//   bf16: v_mfma_f32_16x16x32_bf16  (one 16-byte fragment per lane = 8 bf16 along K)
//   fp32: v_mfma_f32_16x16x4_f32    (one 16-byte fragment per lane = 4 fp32 along K,
//                                     issued as 4 MFMAs)
// Operand convention: lane l supplies row/column (l & 15) and the K-slot group
// g = l >> 4.  Which physical k a (g, slot) pair stands for is free as long as the
// A and B operands agree, so every product below picks the k-assignment that makes
// its loads contiguous.  The accumulator layout is fixed by the hardware:
//   C[row = 4*g + i][col = l & 15]  for i = 0..3.
// A C tile therefore feeds straight into a later product as the K-side operand when
// the other operand uses the "C-permuted" k-assignment (see frag_cperm_*).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nsa {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 16-byte register piece

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// forward softmax: the exponent reference moves only when a column maximum exceeds it by
// more than this (log2 units), so probabilities stay below 2^8 between rescales
constexpr float kLazyRescale = 8.0f;

struct bf16 {  // storage-only tag type for the template parameter
  uint16_t bits;
};

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}
// round-to-nearest-even float -> bf16 bits (NaN kept quiet)
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int kPerFrag = 4;   // elements in one 16-byte fragment
  static constexpr int kKChunk = 16;   // K covered by one fragment across 4 lane groups
  __device__ static float to_f32(float v) { return v; }
  __device__ static float from_f32(float v) { return v; }
};
template <> struct Elem<bf16> {
  static constexpr int kPerFrag = 8;
  static constexpr int kKChunk = 32;
  __device__ static float to_f32(uint16_t v) { return bf16_bits_to_f32(v); }
  __device__ static uint16_t from_f32(float v) { return f32_to_bf16_bits(v); }
};

// storage type of an element
template <typename T> struct Store { typedef T type; };
template <> struct Store<bf16> { typedef uint16_t type; };

// One K-chunk product: acc += A_frag * B_frag over kKChunk k values.
template <typename T> struct Mma;
template <> struct Mma<bf16> {
  __device__ __forceinline__ static f32x4 run(f32x4 acc, uint4 a, uint4 b) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
  }
};
template <> struct Mma<float> {
  __device__ __forceinline__ static f32x4 run(f32x4 acc, uint4 a, uint4 b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
    return acc;
  }
};

// Keys (the reduction dimension of a P*V-type product) covered by one C-derived
// fragment: two C tiles for bf16 (32 keys), one C tile for fp32 (16 keys).
template <typename T> struct CFrag;
template <> struct CFrag<float> {
  static constexpr int kKeys = 16;
  // c0 holds C rows 4g+i of a 16-row tile: used as-is.
  __device__ __forceinline__ static uint4 pack(f32x4 c0, f32x4 /*c1*/) {
    return make_uint4(__float_as_uint(c0[0]), __float_as_uint(c0[1]), __float_as_uint(c0[2]),
                      __float_as_uint(c0[3]));
  }
};
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
// two floats -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

template <> struct CFrag<bf16> {
  static constexpr int kKeys = 32;
  // slots 0..3 <- tile c0 rows 4g+i ; slots 4..7 <- tile c1 rows 16+4g+i
  __device__ __forceinline__ static uint4 pack(f32x4 c0, f32x4 c1) {
    return make_uint4(pack_bf16x2(c0[0], c0[1]), pack_bf16x2(c0[2], c0[3]), pack_bf16x2(c1[0], c1[1]),
                      pack_bf16x2(c1[2], c1[3]));
  }
};

// "C-permuted" storage of a key-major operand ([rows][keys] arrays whose K axis is the
// key axis: V^T, K^T, and the transposed Q / dO row chunks).  The fragment a lane
// needs is the keys {4g..4g+3} and {16+4g..16+4g+3} of a 32-key chunk (CFrag<bf16>);
// storing each 32-key chunk in the order p = 8g + j  <->  key = j < 4 ? 4g + j : 12 + 4g + j
// makes that fragment one 16-byte vector.  fp32 chunks (16 keys, keys 4g..4g+3 per lane)
// need no permutation.
__host__ __device__ __forceinline__ int cperm_pos32(int key) {  // key within its 32-chunk -> position
  return 8 * ((key & 15) >> 2) + (key & 3) + ((key & 16) ? 4 : 0);
}
template <typename T> __device__ __forceinline__ uint4 frag_cperm(const typename Store<T>::type* row, int g);
template <> __device__ __forceinline__ uint4 frag_cperm<float>(const float* row, int g) {
  return *reinterpret_cast<const uint4*>(row + 4 * g);
}
template <> __device__ __forceinline__ uint4 frag_cperm<bf16>(const uint16_t* row, int g) {
  return *reinterpret_cast<const uint4*>(row + 8 * g);
}

// LDS transpose load (ds_read_b64_tr_b16): within each 16-lane group, lanes 4*rho..4*rho+3
// together address row rho (16 consecutive 16-bit elements, 4 per lane) of a 4 x 16
// block and lane j receives column j: {row0[j], row1[j], row2[j], row3[j]}.
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 ld_tr16x4(const uint16_t* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(uint2, v);
}
// Two transpose loads, the second `delta` elements further on: one 8-slot bf16 fragment.
__device__ __forceinline__ uint4 ld_tr_pair(const uint16_t* p, int delta) {
  const uint2 lo = ld_tr16x4(p), hi = ld_tr16x4(p + delta);
  return make_uint4(lo.x, lo.y, hi.x, hi.y);
}

// Fragment-native operand layouts of a [R][C] matrix (R on the time axis, C features;
// R a multiple of 64, C of 32): every 16-byte MFMA fragment of a 64-lane wave sits at
// lane * 16 bytes of one contiguous 1 KB tile, so a fragment load is one coalesced
// 1 KB request instead of 16 row pieces.
//  rowfrag: A/B operand whose rows are time (16 per tile) and whose K slots run along
//           the features (kKChunk per tile; lane g*16 + r holds features g*kPerFrag..).
//  colfrag: operand whose rows are features (16 per tile) and whose K slots run along
//           time in the C-permuted order of a CFrag chunk (lane g*16 + f holds the
//           kPerFrag times of group g).
template <typename T>
__host__ __device__ __forceinline__ int64_t rowfrag_off(int r, int c, int C) {
  constexpr int EPF = Elem<T>::kPerFrag, KC = Elem<T>::kKChunk;
  return ((((int64_t)(r >> 4) * (C / KC) + c / KC) * 64 + ((c % KC) / EPF) * 16 + (r & 15)) * EPF) + (c % EPF);
}
template <typename T>
__host__ __device__ __forceinline__ int64_t colfrag_off(int r, int c, int C) {
  constexpr int EPF = Elem<T>::kPerFrag, CK = CFrag<T>::kKeys;
  const int p = CK == 32 ? cperm_pos32(r & 31) : (r & 15);
  return ((((int64_t)(r / CK) * (C / 16) + (c >> 4)) * 64 + (p / EPF) * 16 + (c & 15)) * EPF) + (p % EPF);
}
// the lane's fragment of rowfrag tile (row16, kc) / colfrag tile (chunk, fgroup)
template <typename T>
__device__ __forceinline__ uint4 ld_rowfrag(const typename Store<T>::type* m, int row16, int kc, int C, int lane) {
  constexpr int EPF = Elem<T>::kPerFrag, KC = Elem<T>::kKChunk;
  return *reinterpret_cast<const uint4*>(m + (((int64_t)row16 * (C / KC) + kc) * 64 + lane) * EPF);
}
template <typename T>
__device__ __forceinline__ uint4 ld_colfrag(const typename Store<T>::type* m, int chunk, int fg, int C, int lane) {
  constexpr int EPF = Elem<T>::kPerFrag;
  return *reinterpret_cast<const uint4*>(m + (((int64_t)chunk * (C / 16) + fg) * 64 + lane) * EPF);
}

// Standard fragment: 16 contiguous bytes at row[kchunk_base + g * kPerFrag].
template <typename T>
__device__ __forceinline__ uint4 frag_std(const typename Store<T>::type* row, int g) {
  return *reinterpret_cast<const uint4*>(row + g * Elem<T>::kPerFrag);
}


__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Direct global -> LDS copy (global_load_lds_dwordx4): every lane reads 16 bytes at
// its own `src` and lane l's bytes land at lds_base + 16 l.  lds_base must be
// wave-uniform and 16-byte aligned; the copy completes with the wave's vmcnt.  The
// explicit address-space casts keep the host-side instantiation of the calling
// kernels valid.
__device__ __forceinline__ void copy16_to_lds(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)(src),
                                   (__attribute__((address_space(3))) void*)(lds_base), 16, 0, 0);
}

// The same copy issued from inline assembly, so that the compiler's wait insertion does
// not see it.  The compiler cannot tell which LDS bytes a direct-to-LDS copy writes, so
// it makes every later LDS read wait for every such copy in flight, which would stall a
// tile's reads on the copy of the next tile.  A caller of this variant waits for the copy
// itself (s_waitcnt vmcnt(0)) before the barrier that publishes the data.
__device__ __forceinline__ void copy16_to_lds_async(const void* src, void* lds_base) {
  // wave-uniform by contract: taken from the first lane so that it lives in an SGPR
  const uint32_t lds =
      __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)((__attribute__((address_space(3))) char*)(lds_base)));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "s"(lds) : "memory", "m0");
}

// Orders a wave's LDS stores before its later LDS loads of other lanes' data: waits
// for the wave's LDS operations only (lgkmcnt(0), vmcnt / expcnt left at their
// maximum), so global loads and stores stay in flight.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_wave_barrier();
}

// Waits until at most N of the wave's vector-memory operations are outstanding (they
// complete in issue order for loads), leaving lgkmcnt / expcnt unconstrained; gfx9
// s_waitcnt encoding: vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8].
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Store 4 consecutive values (one C-tile column slice) as T.
template <typename T> __device__ __forceinline__ void store4(typename Store<T>::type* p, f32x4 v);
template <> __device__ __forceinline__ void store4<float>(float* p, f32x4 v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
template <> __device__ __forceinline__ void store4<bf16>(uint16_t* p, f32x4 v) {
  *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
}
// The values 4 consecutive T elements would hold once stored (rounded to T).
template <typename T> __device__ __forceinline__ f32x4 round4(f32x4 v);
template <> __device__ __forceinline__ f32x4 round4<float>(f32x4 v) { return v; }
template <> __device__ __forceinline__ f32x4 round4<bf16>(f32x4 v) {
  return f32x4{bf16_bits_to_f32(f32_to_bf16_bits(v[0])), bf16_bits_to_f32(f32_to_bf16_bits(v[1])),
               bf16_bits_to_f32(f32_to_bf16_bits(v[2])), bf16_bits_to_f32(f32_to_bf16_bits(v[3]))};
}

// 4 consecutive T values in storage form (8 bytes bf16, 16 bytes fp32): loaded early,
// converted and added later.
template <typename T> struct Raw4 { typedef uint4 type; };
template <> struct Raw4<bf16> { typedef uint2 type; };
template <typename T>
__device__ __forceinline__ typename Raw4<T>::type load4_raw(const typename Store<T>::type* p) {
  return *reinterpret_cast<const typename Raw4<T>::type*>(p);
}
__device__ __forceinline__ f32x4 raw4_f32(const uint4& v) {
  return f32x4{__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w)};
}
__device__ __forceinline__ f32x4 raw4_f32(const uint2& v) {
  return f32x4{__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.y << 16),
               __uint_as_float(v.y & 0xffff0000u)};
}

// Load 4 consecutive T values as fp32.
template <typename T> __device__ __forceinline__ f32x4 load4(const typename Store<T>::type* p);
template <> __device__ __forceinline__ f32x4 load4<float>(const float* p) {
  const float4 v = *reinterpret_cast<const float4*>(p);
  return f32x4{v.x, v.y, v.z, v.w};
}
template <> __device__ __forceinline__ f32x4 load4<bf16>(const uint16_t* p) {
  const uint2 v = *reinterpret_cast<const uint2*>(p);
  return f32x4{__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.y << 16),
               __uint_as_float(v.y & 0xffff0000u)};
}

// p[(e + u) * sd] += v[u] for u < 4, in fp32 and rounded once to T (one vector
// read-modify-write when the four elements are contiguous and aligned).
template <typename T>
__device__ __forceinline__ void add4(typename Store<T>::type* p, int64_t e, int64_t sd, f32x4 v) {
  using S = typename Store<T>::type;
  S* q = p + e * sd;
  if (sd == 1 && (reinterpret_cast<uintptr_t>(q) % (4 * sizeof(S))) == 0) {
    const f32x4 old = load4<T>(q);
    store4<T>(q, old + v);
  } else {
#pragma unroll
    for (int u = 0; u < 4; ++u) q[u * sd] = Elem<T>::from_f32(Elem<T>::to_f32(q[u * sd]) + v[u]);
  }
}

// p[(e + u) * sd] = v[u] for u < 4, rounded to T (one vector store when the four
// elements are contiguous and aligned).
template <typename T>
__device__ __forceinline__ void set4(typename Store<T>::type* p, int64_t e, int64_t sd, f32x4 v) {
  using S = typename Store<T>::type;
  S* q = p + e * sd;
  if (sd == 1 && (reinterpret_cast<uintptr_t>(q) % (4 * sizeof(S))) == 0) {
    store4<T>(q, v);
  } else {
#pragma unroll
    for (int u = 0; u < 4; ++u) q[u * sd] = Elem<T>::from_f32(v[u]);
  }
}

// 2^x on the transcendental unit (v_exp_f32); exp2(-inf) = 0.  Inputs here are <= 0,
// results below the normal range may flush, which the softmax tolerates.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// round(x * y) + r as two rounded operations (never contracted to one fma): with r the
// negated rounded product of a maximum, that maximum maps to exactly 0
__device__ __forceinline__ float mul_add_rounded(float x, float y, float r) {
#pragma clang fp contract(off)
  return x * y + r;
}

// n / d and n % d for 0 <= n < 2^31, branch-free: q = (n * m) >> s with
// l = ceil(log2 d), s = 31 + l, m = ceil(2^s / d).  m < 2^32 because d > 2^(l-1), and the
// rounding error n (m - 2^s/d) / 2^s < 2^-l <= 1/d never reaches the next integer.
struct IntDiv {
  int d;
  uint32_t m;
  int s;
  __host__ __device__ static IntDiv make(int d_) {
    int l = 0;
    while ((1ll << l) < d_) ++l;
    const uint64_t two_s = 1ull << (31 + l);
    return IntDiv{d_, (uint32_t)((two_s + (uint64_t)d_ - 1) / (uint64_t)d_), 31 + l};
  }
  __device__ __forceinline__ int div(int n) const {
    return (int)(((uint64_t)(uint32_t)n * m) >> s);
  }
  __device__ __forceinline__ int mod(int n) const { return n - div(n) * d; }
};

// Value of lane L ^ OFF of a wave64 (OFF a power of two below 64) without the LDS
// crossbar: v_permlane32_swap / v_permlane16_swap for 32 and 16 (each swap returns the
// other half's values in the result the lane's own half does not keep), DPP row_ror:8
// for 8, row_ror:4 or :12 by lane for 4, quad_perm for 2 and 1.  Equal to
// __shfl_xor(x, OFF) on every lane.
template <int OFF>
__device__ __forceinline__ uint32_t lane_xor_u32(uint32_t x) {
  static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8 || OFF == 16 || OFF == 32, "lane offset");
  const int lane = threadIdx.x & 63;
  if constexpr (OFF == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (lane & 32) ? r[0] : r[1];
  } else if constexpr (OFF == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (lane & 16) ? r[0] : r[1];
  } else if constexpr (OFF == 8) {
    return __builtin_amdgcn_update_dpp(0u, x, 0x128, 0xF, 0xF, false);  // row_ror:8
  } else if constexpr (OFF == 4) {
    const uint32_t lo = __builtin_amdgcn_update_dpp(0u, x, 0x124, 0xF, 0xF, false);  // row_ror:4
    const uint32_t hi = __builtin_amdgcn_update_dpp(0u, x, 0x12C, 0xF, 0xF, false);  // row_ror:12
    return (lane & 4) ? lo : hi;
  } else if constexpr (OFF == 2) {
    return __builtin_amdgcn_update_dpp(0u, x, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  } else {
    return __builtin_amdgcn_update_dpp(0u, x, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  }
}
template <int OFF>
__device__ __forceinline__ float lane_xor(float x) {
  return __uint_as_float(lane_xor_u32<OFF>(__float_as_uint(x)));
}
template <int OFF>
__device__ __forceinline__ int lane_xor(int x) {
  return (int)lane_xor_u32<OFF>((uint32_t)x);
}
// max / sum over the four lanes sharing (l & 15), lane swaps instead of LDS-crossbar
// shuffles (same pairing order as __shfl_xor with 16, then 32)
__device__ __forceinline__ float wave_max16(float v) {
  v = fmaxf(v, lane_xor<16>(v));
  v = fmaxf(v, lane_xor<32>(v));
  return v;
}
__device__ __forceinline__ float wave_sum16(float v) {
  v += lane_xor<16>(v);
  v += lane_xor<32>(v);
  return v;
}

// xor butterfly over 32, 16, 8, 4, 2, 1: every lane ends with op folded over the wave,
// pairs combined in exactly the order of the __shfl_xor loop over the same offsets
template <typename T, typename F>
__device__ __forceinline__ T wave_butterfly(T x, F op) {
  x = op(x, lane_xor<32>(x));
  x = op(x, lane_xor<16>(x));
  x = op(x, lane_xor<8>(x));
  x = op(x, lane_xor<4>(x));
  x = op(x, lane_xor<2>(x));
  x = op(x, lane_xor<1>(x));
  return x;
}

}  // namespace nsa
