// Backward row statistics, computed by the dQ kernels for their own query columns:
//   delta = sum_d O[d] * dO[d]   (fp32; or the caller's precomputed sums, delta_in)
//   lse2  = (M + L) * log2(e)    (+inf when L = -inf: the row saw no key, every p is 0)
//   gate  = row_gate[row]        (1 without a row gate)
// With a row gate g the branch's output gradient is g dO: dP, D and dS all scale by g,
// so the kernels keep D = sum_d O dO unscaled, multiply dQ by g at the end and the
// probabilities of dK / dV by g per row; row_dot (when given) receives that unscaled D,
// the gate's own gradient.
// The dQ kernels use them directly and store them (AttnArgs::rstat) for the dK/dV
// kernel, which runs after dQ on the same stream (one pass over O fewer than a separate statistics
// kernel: dO is already in the dQ kernel's registers).
#pragma once
#include "nsa_attn.h"
#include "nsa_device.h"

namespace nsa {

// Lane (c16, g4) of a 16-column subtile holds dO[col][kc * KC + g4 * EPF + u] in dof[kc]
// (the MFMA operand layout); it reads O at the same positions, and the four lane groups
// of a column are summed by two xor steps.  Stores from lane group 0 of valid columns.
template <typename T, int NVC>
__device__ __forceinline__ void dq_row_stats(const AttnArgs& a, int b, int colh, int colt, bool colv,
                                             const uint4 (&dof)[NVC], int g4, int64_t srow, float& l2,
                                             float& dl, float& gate) {
  using S = typename Store<T>::type;
  constexpr int EPF = Elem<T>::kPerFrag;
  constexpr int KC = Elem<T>::kKChunk;
  if (a.delta_in) {  // the caller's row sums: O is not read
    dl = colv ? a.delta_in[srow] : 0.f;
  } else {
    const S* op = reinterpret_cast<const S*>(a.o) + b * a.so_b + (int64_t)colh * a.so_h + (int64_t)colt * a.so_t;
    float acc = 0.f;
#pragma unroll
    for (int kc = 0; kc < NVC; ++kc) {
      const uint4 ov = colv ? *reinterpret_cast<const uint4*>(op + kc * KC + g4 * EPF) : make_uint4(0, 0, 0, 0);
      const S* o = reinterpret_cast<const S*>(&ov);
      const S* d = reinterpret_cast<const S*>(&dof[kc]);
#pragma unroll
      for (int u = 0; u < EPF; ++u) acc = fmaf(Elem<T>::to_f32(o[u]), Elem<T>::to_f32(d[u]), acc);
    }
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    dl = colv ? acc : 0.f;
  }
  l2 = INFINITY;
  gate = (a.row_gate && colv) ? a.row_gate[srow] : 1.f;
  if (colv) {
    const float L = a.L[b * a.sl_b + (int64_t)colh * a.sl_h + (int64_t)colt * a.sl_t];
    const float M = a.M[b * a.sm_b + (int64_t)colh * a.sm_h + (int64_t)colt * a.sm_t];
    l2 = L == -INFINITY ? INFINITY : (M + L) * kLog2e;
    if (g4 == 0) {
      const int hh = colh % a.hpg;  // the head within its group
      a.rstat[((int64_t)(b * a.G + colh / a.hpg) * a.Tq + colt) * a.hpg + hh] = make_float4(l2, dl, gate, 0.f);
      if (a.row_dot) a.row_dot[srow] = dl;
    }
  }
}

}  // namespace nsa
