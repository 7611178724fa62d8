// Backward attention for the three NSA branches on gfx950, split FlashAttention-2
// style into a query-major dQ kernel and a key-major dK/dV kernel.  Neither uses
// floating-point atomics: each dQ row and each dK/dV row has exactly one owner, and
// where one key tile's queries are spread over several work items (compression,
// selection) the items write fp32 partials that a reduce kernel sums in a fixed
// order.  Results are therefore bit-reproducible run to run.
//
// Math (reference backward, nsa/kernels.py:1303-1530): with s = scale * q.k,
//   p  = exp(s - M - L)                    (saved forward statistics)
//   dP = dO . v,   D = rowsum(O * dO),   dS = p * (dP - D)
//   dQ = scale * dS . K      dK = scale * dS^T . Q      dV = p^T . dO
#pragma once
#include "nsa_attn.h"
#include "nsa_device.h"

namespace nsa {

// ============================== dQ (query-major) ===============================
template <typename T, int DK, int DV, int BR>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(AttnArgs a) {
  using S = typename Store<T>::type;
  constexpr int EPF = Elem<T>::kPerFrag;
  constexpr int KC = Elem<T>::kKChunk;
  constexpr int NKC = DK / KC;
  constexpr int NVC = DV / KC;
  constexpr int KP = DK + EPF;
  constexpr int NP = 64 + EPF;
  constexpr int VP = DV + EPF;
  constexpr int CK = CFrag<T>::kKeys;
  constexpr int CT = CK / 16;
  static_assert(DK % KC == 0 && DV % KC == 0, "head dims");

  __shared__ __attribute__((aligned(16))) S Ks[64 * KP];   // K rows   [key][d]
  __shared__ __attribute__((aligned(16))) S KnS[DK * NP];  // K^T      [d][key]
  __shared__ __attribute__((aligned(16))) S Vns[64 * VP];  // V rows   [key][dv]
  __shared__ int s_be[64];
  __shared__ int s_misc[4];
  __shared__ int s_list[BR == kSelection ? kSelListMax : 1];
  __shared__ int s_union[BR == kSelection ? kSelMaxBlocks : 1];
  __shared__ uint32_t s_bits[BR == kSelection ? kSelMaxBlocks / 32 : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g4 = lane >> 4;
  const int c16 = lane & 15;
  const int bg = blockIdx.y;
  const int b = bg / a.G;
  const int grp = bg % a.G;
  const int hpg = a.hpg;
  const int ncols = a.Tq * hpg;
  const int col_base = blockIdx.x * kDqCols;
  const int t_first = col_base / hpg;
  const int t_last = min(a.Tq - 1, (col_base + kDqCols - 1) / hpg);
  const float scale2 = a.scale * kLog2e;

  const S* kt = reinterpret_cast<const S*>(a.kt) + (int64_t)bg * a.Tp * DK;
  const S* kn = reinterpret_cast<const S*>(a.kn) + (int64_t)bg * DK * a.Tp;
  const S* vn = reinterpret_cast<const S*>(a.vn) + (int64_t)bg * a.Tp * DV;

  // one 16-column subtile per wave
  const int f0 = col_base + wave * 16;
  const int f = f0 + c16;
  const bool colv = f < ncols;
  const int colt = colv ? f / hpg : 0;
  const int colh = colv ? grp * hpg + f % hpg : 0;
  const int sub_t0 = f0 / hpg;
  const int sub_t1 = f0 < ncols ? min(a.Tq - 1, (f0 + 15) / hpg) : -1;
  uint4 qf[NKC], dof[NVC];
  {
    const S* qp = reinterpret_cast<const S*>(a.q) + b * a.sq_b + (int64_t)colh * a.sq_h + (int64_t)colt * a.sq_t;
    const S* dp = reinterpret_cast<const S*>(a.dout) + b * a.sdo_b + (int64_t)colh * a.sdo_h +
                  (int64_t)colt * a.sdo_t;
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc)
      qf[kc] = colv ? *reinterpret_cast<const uint4*>(qp + kc * KC + g4 * EPF) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int kc = 0; kc < NVC; ++kc)
      dof[kc] = colv ? *reinterpret_cast<const uint4*>(dp + kc * KC + g4 * EPF) : make_uint4(0, 0, 0, 0);
  }
  const int64_t srow = ((int64_t)b * a.H + colh) * a.Tq + colt;
  const float l2 = colv ? a.lse2[srow] : INFINITY;
  const float dl = colv ? a.delta[srow] : 0.f;

  f32x4 dqa[DK / 16];
#pragma unroll
  for (int j = 0; j < DK / 16; ++j) dqa[j] = zero4();

  int ntiles = 0, key_lo = 0, nsubblk = 1;
  if (BR == kSliding) {
    key_lo = max(0, t_first - a.window + 1) & ~15;
    const int hi = min(t_last, a.Tkv - 1);
    ntiles = hi >= key_lo ? (hi - key_lo) / 64 + 1 : 0;
  } else if (BR == kCompression) {
    if (tid == 0) s_misc[0] = 0;
    __syncthreads();
    int mx = 0;
    for (int i = tid; i < a.Tkv; i += 256)
      if (a.block_ends[i] <= t_last) mx = i + 1;
    if (mx) atomicMax(&s_misc[0], mx);
    __syncthreads();
    ntiles = (s_misc[0] + 63) / 64;
  } else {
    const int nt = t_last - t_first + 1;
    const int total = nt * a.nslots;
    const int nwords = (a.nblk + 31) / 32;
    for (int i = tid; i < nwords; i += 256) s_bits[i] = 0;
    __syncthreads();
    const int* selrow = a.sel + ((int64_t)bg * a.Tq + t_first) * a.nslots;
    for (int i = tid; i < total; i += 256) {
      const int v = selrow[i];
      s_list[i] = v;
      if (v >= 0) atomicOr(&s_bits[v >> 5], 1u << (v & 31));
    }
    __syncthreads();
    if (tid == 0) {
      int n = 0;
      for (int w = 0; w < nwords; ++w) {
        uint32_t bits = s_bits[w];
        while (bits) {
          const int bit = __builtin_ctz(bits);
          bits &= bits - 1;
          s_union[n++] = w * 32 + bit;
        }
      }
      s_misc[0] = n;
    }
    __syncthreads();
    nsubblk = (a.lprime + 63) / 64;
    ntiles = s_misc[0] * nsubblk;
  }

  for (int it = 0; it < ntiles; ++it) {
    int key0, blk_lo = 0, blk_hi = 0;
    if (BR == kSliding) {
      key0 = key_lo + it * 64;
    } else if (BR == kCompression) {
      key0 = it * 64;
    } else {
      const int blk = s_union[it / nsubblk];
      blk_lo = blk * a.lprime;
      blk_hi = min(blk_lo + a.lprime, a.Tkv);
      key0 = blk_lo + (it % nsubblk) * 64;
      if ((a.causal && key0 > t_last) || key0 >= blk_hi) continue;
    }
    for (int c = tid; c < 64 * (DK / EPF); c += 256) {
      const int r = c / (DK / EPF);
      const int e = (c % (DK / EPF)) * EPF;
      *reinterpret_cast<uint4*>(&Ks[r * KP + e]) = *reinterpret_cast<const uint4*>(kt + (int64_t)(key0 + r) * DK + e);
    }
    for (int c = tid; c < DK * (64 / EPF); c += 256) {
      const int r = c / (64 / EPF);
      const int e = (c % (64 / EPF)) * EPF;
      *reinterpret_cast<uint4*>(&KnS[r * NP + e]) = *reinterpret_cast<const uint4*>(kn + (int64_t)r * a.Tp + key0 + e);
    }
    for (int c = tid; c < 64 * (DV / EPF); c += 256) {
      const int r = c / (DV / EPF);
      const int e = (c % (DV / EPF)) * EPF;
      *reinterpret_cast<uint4*>(&Vns[r * VP + e]) = *reinterpret_cast<const uint4*>(vn + (int64_t)(key0 + r) * DV + e);
    }
    if (BR == kCompression && tid < 64) {
      const int key = key0 + tid;
      s_be[tid] = key < a.Tkv ? a.block_ends[key] : 0x7fffffff;
    }
    __syncthreads();

    bool active;
    bool colsel = false;
    if (BR == kSliding) {
      active = sub_t1 >= 0 && key0 <= sub_t1 && key0 + 63 > sub_t0 - a.window;
    } else if (BR == kCompression) {
      int be_min = s_be[lane];
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) be_min = min(be_min, __shfl_xor(be_min, o));
      active = sub_t1 >= 0 && be_min <= sub_t1;
    } else {
      if (colv && (!a.causal || key0 <= colt)) {
        const int* lst = &s_list[(colt - t_first) * a.nslots];
        const int blk = blk_lo / a.lprime;
        for (int j = 0; j < a.nslots; ++j) {
          const int v = lst[j];
          if (v == blk) colsel = true;
          if (v < 0 || v >= blk) break;
        }
      }
      active = __ballot(colsel) != 0ull;
    }

    if (active) {
      f32x4 st[4], dp[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        st[ks] = zero4();
        dp[ks] = zero4();
        const S* krow = &Ks[(ks * 16 + c16) * KP];
        const S* vrow = &Vns[(ks * 16 + c16) * VP];
#pragma unroll
        for (int kc = 0; kc < NKC; ++kc) st[ks] = Mma<T>::run(st[ks], frag_std<T>(krow + kc * KC, g4), qf[kc]);
#pragma unroll
        for (int kc = 0; kc < NVC; ++kc) dp[ks] = Mma<T>::run(dp[ks], frag_std<T>(vrow + kc * KC, g4), dof[kc]);
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = key0 + ks * 16 + 4 * g4 + i;
          bool ok;
          if (BR == kSliding) {
            ok = colv && key <= colt && key > colt - a.window && key < a.Tkv;
          } else if (BR == kCompression) {
            ok = colv && s_be[ks * 16 + 4 * g4 + i] <= colt;
          } else {
            ok = colsel && (!a.causal || key <= colt) && key < blk_hi;
          }
          const float p = ok ? exp2f(st[ks][i] * scale2 - l2) : 0.f;
          st[ks][i] = p * (dp[ks][i] - dl);  // dS^T
        }
      }
#pragma unroll
      for (int kc2 = 0; kc2 < 64 / CK; ++kc2) {
        const uint4 sf = CFrag<T>::pack(st[kc2 * CT], st[kc2 * CT + CT - 1]);
#pragma unroll
        for (int j = 0; j < DK / 16; ++j) {
          const uint4 kf = frag_cperm<T>(&KnS[(j * 16 + c16) * NP + kc2 * CK], g4);
          dqa[j] = Mma<T>::run(dqa[j], kf, sf);
        }
      }
    }
    __syncthreads();
  }

  if (colv) {
    S* dqp = reinterpret_cast<S*>(a.dq) + b * a.sdq_b + (int64_t)colh * a.sdq_h + (int64_t)colt * a.sdq_t;
#pragma unroll
    for (int j = 0; j < DK / 16; ++j) store4<T>(dqp + j * 16 + 4 * g4, dqa[j] * a.scale);
  }
}

template <typename T, int DK, int DV, int BR>
void launch_attn_bwd_dq(const AttnArgs& a, hipStream_t s) {
  dim3 grid((a.Tq * a.hpg + kDqCols - 1) / kDqCols, a.B * a.G);
  hipLaunchKernelGGL((attn_bwd_dq_kernel<T, DK, DV, BR>), grid, dim3(256), 0, s, a);
}

// ============================== dK / dV (key-major) =============================
// A workgroup owns 64 keys (16 per wave) and walks the query rows that can see
// them in chunks of 32 (timestep, head) rows staged in LDS both row-major (operand
// of S = Q K^T and dP = dO V^T) and transposed (operand of dK^T += Q^T dS and
// dV^T += dO^T P, whose reduction runs over the rows).
template <typename T, int DK, int DV, int BR>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_kernel(AttnArgs a) {
  using S = typename Store<T>::type;
  constexpr int EPF = Elem<T>::kPerFrag;
  constexpr int KC = Elem<T>::kKChunk;
  constexpr int NKC = DK / KC;
  constexpr int NVC = DV / KC;
  constexpr int RC = kRowChunk;  // 32 rows
  constexpr int QP = DK + EPF;
  constexpr int OP = DV + EPF;
  constexpr int RP = RC + EPF;
  constexpr int CK = CFrag<T>::kKeys;
  constexpr int CT = CK / 16;
  static_assert(RC % CK == 0, "row chunk");

  __shared__ __attribute__((aligned(16))) S Qs[RC * QP];
  __shared__ __attribute__((aligned(16))) S QTs[DK * RP];
  __shared__ __attribute__((aligned(16))) S Os[RC * OP];
  __shared__ __attribute__((aligned(16))) S OTs[DV * RP];
  __shared__ int s_t[RC];
  __shared__ int s_h[RC];
  __shared__ float s_l2[RC];
  __shared__ float s_dl[RC];
  __shared__ int s_be[64];
  __shared__ int s_misc[4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g4 = lane >> 4;
  const int c16 = lane & 15;
  const int bg = blockIdx.y;
  const int b = bg / a.G;
  const int grp = bg % a.G;
  const int hpg = a.hpg;
  const float scale2 = a.scale * kLog2e;
  const int item = blockIdx.x;

  // ---- decode the work item: key tile + range of rows ----
  int key0, blk_hi = a.Tkv;
  int64_t f_lo, f_hi;        // flattened row range (row index -> (t, head))
  const int* tlist = nullptr;  // selection: row f -> t = tlist[f / hpg]
  if (BR == kSliding) {
    key0 = item * 64;
    const int t_lo = key0;
    const int t_hi = min(a.Tq - 1, key0 + 63 + a.window - 1);
    f_lo = (int64_t)t_lo * hpg;
    f_hi = t_hi >= t_lo ? (int64_t)(t_hi + 1) * hpg : f_lo;
  } else if (BR == kCompression) {
    const int nseg = (a.Tq + kSegT - 1) / kSegT;
    const int tile = item / nseg, seg = item % nseg;
    key0 = tile * 64;
    if (tid < 64) {
      const int key = key0 + tid;
      s_be[tid] = key < a.Tkv ? a.block_ends[key] : 0x7fffffff;
    }
    __syncthreads();
    int be_min = s_be[lane];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) be_min = min(be_min, __shfl_xor(be_min, o));
    const int t_lo = max(seg * kSegT, max(be_min, 0));
    const int t_hi = min(a.Tq, (seg + 1) * kSegT);
    f_lo = (int64_t)t_lo * hpg;
    f_hi = t_hi > t_lo ? (int64_t)t_hi * hpg : f_lo;
  } else {
    const int nsubblk = (a.lprime + 63) / 64;
    const int sidx = item / nsubblk, sub = item % nsubblk;
    const int* so = a.seg_off + (int64_t)bg * (a.nblk + 1);
    if (sidx >= so[a.nblk]) return;  // beyond this group's work list (uniform)
    int lo = 0, hi = a.nblk;         // largest j with so[j] <= sidx
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (so[mid] <= sidx) lo = mid;
      else hi = mid;
    }
    const int j = lo;
    const int k = sidx - so[j];
    const int* co = a.csr_off + (int64_t)bg * (a.nblk + 1);
    const int e_lo = co[j] + k * kSegT;
    const int e_hi = min(co[j + 1], e_lo + kSegT);
    tlist = a.csr_t + (int64_t)bg * a.Tq * a.nslots;
    key0 = j * a.lprime + sub * 64;
    blk_hi = min(j * a.lprime + a.lprime, a.Tkv);
    f_lo = (int64_t)e_lo * hpg;
    f_hi = (int64_t)e_hi * hpg;
    if (key0 >= blk_hi) return;  // sub-tile past the sequence end: nothing to own
  }

  // ---- this wave's 16 keys: K and V rows as B operands, kept in registers ----
  const S* kt = reinterpret_cast<const S*>(a.kt) + (int64_t)bg * a.Tp * DK;
  const S* vn = reinterpret_cast<const S*>(a.vn) + (int64_t)bg * a.Tp * DV;
  const int kw0 = key0 + wave * 16;
  const int mykey = kw0 + c16;
  uint4 kf[NKC], vf[NVC];
#pragma unroll
  for (int kc = 0; kc < NKC; ++kc) kf[kc] = *reinterpret_cast<const uint4*>(kt + (int64_t)mykey * DK + kc * KC + g4 * EPF);
#pragma unroll
  for (int kc = 0; kc < NVC; ++kc) vf[kc] = *reinterpret_cast<const uint4*>(vn + (int64_t)mykey * DV + kc * KC + g4 * EPF);
  int mybe = 0x7fffffff, wave_be_min = 0x7fffffff;
  if (BR == kCompression) {
    mybe = s_be[wave * 16 + c16];
    wave_be_min = mybe;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) wave_be_min = min(wave_be_min, __shfl_xor(wave_be_min, o));
  }

  f32x4 dka[DK / 16], dva[DV / 16];
#pragma unroll
  for (int j = 0; j < DK / 16; ++j) dka[j] = zero4();
#pragma unroll
  for (int j = 0; j < DV / 16; ++j) dva[j] = zero4();

  const S* qbase = reinterpret_cast<const S*>(a.q);
  const S* obase = reinterpret_cast<const S*>(a.dout);

  for (int64_t fc = f_lo; fc < f_hi; fc += RC) {
    // row bookkeeping
    if (tid < RC) {
      const int64_t f = fc + tid;
      int t = -1, h = 0;
      if (f < f_hi) {
        const int64_t e = f / hpg;
        h = grp * hpg + (int)(f % hpg);
        t = tlist ? tlist[e] : (int)e;
      }
      s_t[tid] = t;
      s_h[tid] = h;
      if (t >= 0) {
        const int64_t srow = ((int64_t)b * a.H + h) * a.Tq + t;
        s_l2[tid] = a.lse2[srow];
        s_dl[tid] = a.delta[srow];
      } else {
        s_l2[tid] = INFINITY;
        s_dl[tid] = 0.f;
      }
    }
    __syncthreads();
    // stage Q and dO rows, row-major and transposed
    for (int c = tid; c < RC * (DK / EPF); c += 256) {
      const int r = c / (DK / EPF);
      const int e = (c % (DK / EPF)) * EPF;
      const int t = s_t[r];
      uint4 v = make_uint4(0, 0, 0, 0);
      if (t >= 0) v = *reinterpret_cast<const uint4*>(qbase + b * a.sq_b + (int64_t)s_h[r] * a.sq_h + (int64_t)t * a.sq_t + e);
      *reinterpret_cast<uint4*>(&Qs[r * QP + e]) = v;
      const S* vs = reinterpret_cast<const S*>(&v);
#pragma unroll
      for (int u = 0; u < EPF; ++u) QTs[(e + u) * RP + r] = vs[u];
    }
    for (int c = tid; c < RC * (DV / EPF); c += 256) {
      const int r = c / (DV / EPF);
      const int e = (c % (DV / EPF)) * EPF;
      const int t = s_t[r];
      uint4 v = make_uint4(0, 0, 0, 0);
      if (t >= 0) v = *reinterpret_cast<const uint4*>(obase + b * a.sdo_b + (int64_t)s_h[r] * a.sdo_h + (int64_t)t * a.sdo_t + e);
      *reinterpret_cast<uint4*>(&Os[r * OP + e]) = v;
      const S* vs = reinterpret_cast<const S*>(&v);
#pragma unroll
      for (int u = 0; u < EPF; ++u) OTs[(e + u) * RP + r] = vs[u];
    }
    __syncthreads();

    // coarse skip: rows are in ascending t, so the chunk spans [t_min, t_max]
    int t_min = s_t[0], t_max = -1;
    for (int r = RC - 1; r >= 0; --r) {
      if (s_t[r] >= 0) {
        t_max = s_t[r];
        break;
      }
    }
    bool active;
    if (BR == kSliding) active = t_max >= 0 && kw0 <= t_max && kw0 + 15 > t_min - a.window;
    else if (BR == kCompression) active = t_max >= 0 && wave_be_min <= t_max;
    else active = t_max >= 0 && (!a.causal || kw0 <= t_max) && kw0 < blk_hi;

    if (active) {
      f32x4 pt[RC / 16], dst[RC / 16];
#pragma unroll
      for (int rs = 0; rs < RC / 16; ++rs) {
        f32x4 sacc = zero4(), pacc = zero4();
        const S* qrow = &Qs[(rs * 16 + c16) * QP];
        const S* orow = &Os[(rs * 16 + c16) * OP];
#pragma unroll
        for (int kc = 0; kc < NKC; ++kc) sacc = Mma<T>::run(sacc, frag_std<T>(qrow + kc * KC, g4), kf[kc]);
#pragma unroll
        for (int kc = 0; kc < NVC; ++kc) pacc = Mma<T>::run(pacc, frag_std<T>(orow + kc * KC, g4), vf[kc]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = rs * 16 + 4 * g4 + i;
          const int t = s_t[r];
          bool ok;
          if (BR == kSliding) ok = t >= 0 && mykey <= t && mykey > t - a.window && mykey < a.Tkv;
          else if (BR == kCompression) ok = t >= 0 && mybe <= t;
          else ok = t >= 0 && (!a.causal || mykey <= t) && mykey < blk_hi;
          const float p = ok ? exp2f(sacc[i] * scale2 - s_l2[r]) : 0.f;
          pt[rs][i] = p;
          dst[rs][i] = p * (pacc[i] - s_dl[r]);
        }
      }
#pragma unroll
      for (int kc2 = 0; kc2 < RC / CK; ++kc2) {
        const uint4 pf = CFrag<T>::pack(pt[kc2 * CT], pt[kc2 * CT + CT - 1]);
        const uint4 sf = CFrag<T>::pack(dst[kc2 * CT], dst[kc2 * CT + CT - 1]);
#pragma unroll
        for (int j = 0; j < DV / 16; ++j)
          dva[j] = Mma<T>::run(dva[j], frag_cperm<T>(&OTs[(j * 16 + c16) * RP + kc2 * CK], g4), pf);
#pragma unroll
        for (int j = 0; j < DK / 16; ++j)
          dka[j] = Mma<T>::run(dka[j], frag_cperm<T>(&QTs[(j * 16 + c16) * RP + kc2 * CK], g4), sf);
      }
    }
    __syncthreads();
  }

  // ---- write back: lane holds dK^T[d = 16j + 4*g4 + i][key = mykey] ----
  if (BR == kSliding) {
    if (mykey < a.Tkv) {
      S* dkp = reinterpret_cast<S*>(a.dk) + b * a.sdk_b + grp * a.sdk_g + (int64_t)mykey * a.sdk_t;
      S* dvp = reinterpret_cast<S*>(a.dv) + b * a.sdv_b + grp * a.sdv_g + (int64_t)mykey * a.sdv_t;
#pragma unroll
      for (int j = 0; j < DK / 16; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          S* p = dkp + (int64_t)(j * 16 + 4 * g4 + i) * a.sdk_d;
          *p = Elem<T>::from_f32(Elem<T>::to_f32(*p) + dka[j][i] * a.scale);
        }
#pragma unroll
      for (int j = 0; j < DV / 16; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          S* p = dvp + (int64_t)(j * 16 + 4 * g4 + i) * a.sdv_d;
          *p = Elem<T>::from_f32(Elem<T>::to_f32(*p) + dva[j][i]);
        }
    }
  } else {
    float* pp = a.partial + ((int64_t)bg * a.items_per_bg + item) * 64 * (DK + DV) +
                (int64_t)(wave * 16 + c16) * (DK + DV);
#pragma unroll
    for (int j = 0; j < DK / 16; ++j) {
      const f32x4 v = dka[j] * a.scale;
      *reinterpret_cast<float4*>(pp + j * 16 + 4 * g4) = make_float4(v[0], v[1], v[2], v[3]);
    }
#pragma unroll
    for (int j = 0; j < DV / 16; ++j)
      *reinterpret_cast<float4*>(pp + DK + j * 16 + 4 * g4) = make_float4(dva[j][0], dva[j][1], dva[j][2], dva[j][3]);
  }
}

template <typename T, int DK, int DV, int BR>
void launch_attn_bwd_dkdv(const AttnArgs& a, hipStream_t s) {
  int items;
  if (BR == kSliding) items = (a.Tkv + 63) / 64;
  else items = a.items_per_bg;
  if (items <= 0) return;
  dim3 grid(items, a.B * a.G);
  hipLaunchKernelGGL((attn_bwd_dkdv_kernel<T, DK, DV, BR>), grid, dim3(256), 0, s, a);
}

}  // namespace nsa
