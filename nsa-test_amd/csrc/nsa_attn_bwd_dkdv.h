// dK / dV for the three NSA branches on gfx950 (key-major).
//
// A work item owns 128 keys (selection: one 64-key sub-block) of one (batch, KV
// group) -- 16 keys per wave, held in
// registers as MFMA B operands -- and one segment of the query rows that can see them
// (rows are (timestep, head) pairs of the group).  The rows are walked in chunks of
// RC rows, staged in LDS row-major (operand of S = Q K^T and dP = dO V^T) and
// transposed (operand of dK^T += Q^T dS and dV^T += dO^T P, whose reduction runs over
// the rows).  The next chunk is loaded into registers while the current one is
// computed.  bf16 stages only the row-major rows and reads the transposed operands with
// the LDS transpose load; fp32 stages a transposed copy as well.
// fp32 staging threads own pairs of adjacent rows, so every transposed LDS write stores
// two rows at once, and the transposed row pitch (RC + 4) keeps those writes free of
// bank conflicts.
//
// bf16, heads per group a multiple of 16 (a.ds set): the kernel also stores the dS it
// forms (selection: per (timestep, slot) pair; sliding window / compression: per
// (timestep, 32-key chunk) the timestep sees) for the dQ kernel, which then needs no
// S / dP recomputation.  A 16-row subtile is the 16 heads of one head group of one
// entry / timestep; every wave writes its 16 x 16 dS tiles into a per-chunk LDS tile
// ([key][head], the lane's four heads of one key), and after the next chunk's barrier
// each wave stores one whole 1 KB fragment of it, read back with two transpose loads as
// the lane's eight keys of one head: its share of the dQ product's dS^T operand.
//
// Every item writes its fp32 dK/dV partial for its keys; a reduce kernel sums the
// segments of each key tile in a fixed order and accumulates into the caller's dK/dV.
// Direct mode (sliding window with at least kDkdvDirectItems key tiles over all batches
// and groups, so one item per tile still fills the machine): the item's segment is the
// tile's whole query span and it adds its sums into dK/dV itself, with no partials and
// no reduce.  No floating-point atomics: the result is bit-reproducible.
//
// Backward algebra (reference nsa/kernels.py:1303-1530): with s = scale q.k,
//   p = exp(s - M - L),  dS = p (dO.v - D),  dK = scale dS^T Q,  dV = p^T dO.
#pragma once
#include "nsa_attn.h"
#include "nsa_device.h"

namespace nsa {

// keys per dK/dV work item: the l'-aligned 64-key sub-blocks of selection, 128 keys
// (8 waves) otherwise, so each staged query row serves twice as many keys
__host__ __device__ constexpr int dkdv_keys(int br) { return br == kSelection ? 64 : 128; }

// number of query segments of seg timesteps per key tile (sliding and compression items)
__host__ __device__ inline int dkdv_nseg(int br, int Tq, int window, int seg) {
  if (br == kSliding) {
    const int span = min(window + dkdv_keys(kSliding) - 1, Tq + dkdv_keys(kSliding) - 1);
    return (span + seg - 1) / seg;
  }
  return (Tq + seg - 1) / seg;
}

// the two-row transposed store of one staged 16-byte piece
template <typename S> struct PairT;
template <> struct PairT<uint16_t> {
  // element u of rows (r, r+1) -> one dword at dst[(e+u)*RP + r]
  __device__ __forceinline__ static void store(uint16_t* dst, int RP, const uint4& a, const uint4& b) {
    const uint32_t wa[4] = {a.x, a.y, a.z, a.w};
    const uint32_t wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int w = 0; w < 4; ++w) {  // v_perm_b32: bytes 0-3 from wa, 4-7 from wb
      *reinterpret_cast<uint32_t*>(dst + (2 * w) * RP) = __builtin_amdgcn_perm(wb[w], wa[w], 0x05040100u);
      *reinterpret_cast<uint32_t*>(dst + (2 * w + 1) * RP) = __builtin_amdgcn_perm(wb[w], wa[w], 0x07060302u);
    }
  }
};
template <> struct PairT<float> {
  __device__ __forceinline__ static void store(float* dst, int RP, const uint4& a, const uint4& b) {
    *reinterpret_cast<uint2*>(dst + 0 * RP) = make_uint2(a.x, b.x);
    *reinterpret_cast<uint2*>(dst + 1 * RP) = make_uint2(a.y, b.y);
    *reinterpret_cast<uint2*>(dst + 2 * RP) = make_uint2(a.z, b.z);
    *reinterpret_cast<uint2*>(dst + 3 * RP) = make_uint2(a.w, b.w);
  }
};

// bf16 head dims up to 64 are held to 128 VGPRs (one chunk of row prefetch instead of two), so
// that two 8-wave workgroups share a CU: at these sizes the second workgroup's overlap is
// worth more than the deeper prefetch (benchmark configuration 2: 0.128 -> 0.111 ms per
// fwd+bwd step).
template <typename T, int DK, int DV, int BR>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(DK <= 64 && sizeof(typename Store<T>::type) == 2 ? 4 : 1))) void attn_bwd_dkdv_kernel(
    AttnArgs a) {
  using S = typename Store<T>::type;
  constexpr int KEYS = dkdv_keys(BR);  // keys of the item, 16 per wave
  constexpr int NT = 4 * KEYS;         // threads
  constexpr int EPF = Elem<T>::kPerFrag;
  constexpr int KC = Elem<T>::kKChunk;
  constexpr int NKC = DK / KC;
  constexpr int NVC = DV / KC;
  constexpr int RC = sizeof(S) == 4 ? 16 : kRowChunk;  // fp32 stages half the rows (LDS)
  // bf16 row pitches of 32 B more than the row (416 B at dk = 192, 288 B at dv = 128):
  // an odd multiple of 32 B modulo 256 B, so the 16 rows one transposed read touches
  // fall on distinct banks in each half-wave
  constexpr int QP = DK + (sizeof(S) == 2 ? 16 : EPF);
  constexpr int OP = DV + (sizeof(S) == 2 ? 16 : EPF);
  constexpr int RP = RC + (sizeof(S) == 2 ? 8 : 4);  // 16-byte aligned transposed rows
  constexpr int CK = CFrag<T>::kKeys;
  constexpr int CT = CK / 16;
  constexpr int RPAIRS = RC / 2;
  constexpr int QPC = RPAIRS * (DK / EPF);  // two-row pieces of one Q chunk
  constexpr int OPC = RPAIRS * (DV / EPF);
  // bf16: the transposed operands (Q^T, dO^T) are read from the row-major stage with
  // the LDS transpose load (ds_read_b64_tr_b16), so only the row-major stage exists and
  // every staged piece is one 16-byte run of one row (coalesced global reads).
  // fp32: pairs of rows are staged row-major and transposed.
  constexpr bool kTr = sizeof(S) == 2;
  constexpr int QPCS = kTr ? RC * (DK / EPF) : QPC;  // staged pieces per chunk
  constexpr int OPCS = kTr ? RC * (DV / EPF) : OPC;
  constexpr int NQ = (QPCS + NT - 1) / NT;
  constexpr int NO = (OPCS + NT - 1) / NT;
  static_assert(RC % CK == 0, "row chunk");
  // bf16: two LDS stages (one barrier per chunk; about 44 KB at dk = 192, so two
  // workgroups still share a CU).  fp32 keeps one stage (its transposed copy doubles
  // the footprint).
  constexpr int NB = kTr ? 2 : 1;

  __shared__ __attribute__((aligned(16))) S Qs[NB][RC * QP];
  __shared__ __attribute__((aligned(16))) S QTs[NB][kTr ? 8 : DK * RP];
  __shared__ __attribute__((aligned(16))) S Os[NB][RC * OP];
  __shared__ __attribute__((aligned(16))) S OTs[NB][kTr ? 8 : DV * RP];
  // per staged row: timestep (-1 past the item's end), lse2, delta, gate (1 without a row
  // gate); 16-byte aligned so a lane reads its four consecutive rows at once
  __shared__ __attribute__((aligned(16))) int s_t[NB][RC];
  __shared__ __attribute__((aligned(16))) float s_l2[NB][RC];
  __shared__ __attribute__((aligned(16))) float s_dl[NB][RC];
  __shared__ __attribute__((aligned(16))) float s_g[NB][RC];
  __shared__ int s_be[KEYS];
  __shared__ int s_tl[kSegTMax];  // selection: the item's query timesteps
  // stored dS (selection, bf16): the entries' slots and one 16 x 16 transpose tile per
  // wave and row subtile
  constexpr bool kStoreDs = sizeof(S) == 2;
  __shared__ int s_sl[kStoreDs && BR == kSelection ? kSegTMax : 1];
  // [chunk parity][row subtile][64 keys][16 heads]: a chunk's dS tiles, written by the
  // four waves (their 16 keys each) and stored after the next chunk's barrier
  __shared__ __attribute__((aligned(16))) uint16_t s_dst[kStoreDs ? 2 : 1][RC / 16][kStoreDs ? KEYS * 16 : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g4 = lane >> 4;
  const int c16 = lane & 15;
  const int bg = blockIdx.y;
  const int b = bg / a.G;
  const int grp = bg % a.G;
  const int hpg = a.hpg;
  const IntDiv hdiv = IntDiv::make(hpg);
  const float scale2 = a.scale * kLog2e;
  const int item = blockIdx.x;

  // ---- decode the work item: key tile + segment of rows ----
  int key0, blk_hi = a.Tkv;
  int f_lo, f_hi;              // flattened row range (row f -> (t, head))
  int e_base = 0;              // selection: row f -> t = s_tl[f / hpg - e_base]
  int sub = 0;                 // selection: the item's 64-key sub-block of its block
  if (BR == kSliding) {
    const int nseg = dkdv_nseg(kSliding, a.Tq, a.window, a.seg);
    const int tile = item / nseg, seg = item % nseg;
    key0 = tile * KEYS;
    const int t_lo = key0 + seg * a.seg;
    const int t_hi = min(a.Tq, min(key0 + (seg + 1) * a.seg, key0 + KEYS - 1 + a.window));
    f_lo = t_lo * hpg;
    f_hi = t_hi > t_lo ? t_hi * hpg : f_lo;
  } else if (BR == kCompression) {
    const int nseg = dkdv_nseg(kCompression, a.Tq, 0, a.seg);
    const int tile = item / nseg, seg = item % nseg;
    key0 = tile * KEYS;
    if (tid < KEYS) {
      const int key = key0 + tid;
      s_be[tid] = key < a.Tkv ? a.block_ends[key] : 0x7fffffff;
    }
    __syncthreads();
    int be_min = 0x7fffffff;
#pragma unroll
    for (int c = 0; c < KEYS / 64; ++c) be_min = min(be_min, s_be[c * 64 + lane]);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) be_min = min(be_min, __shfl_xor(be_min, o));
    const int t_lo = max(seg * a.seg, max(be_min, 0));
    const int t_hi = min(a.Tq, (seg + 1) * a.seg);
    f_lo = t_lo * hpg;
    f_hi = t_hi > t_lo ? t_hi * hpg : f_lo;
  } else {
    const int nsubblk = (a.lprime + 63) / 64;
    const int sidx = item / nsubblk;
    sub = item % nsubblk;
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
    const int e_lo = co[j] + k * a.seg;
    const int e_hi = min(co[j + 1], e_lo + a.seg);
    key0 = j * a.lprime + sub * 64;
    blk_hi = min(j * a.lprime + a.lprime, a.Tkv);
    f_lo = e_lo * hpg;
    f_hi = e_hi * hpg;
    if (key0 >= blk_hi) return;  // sub-tile past the sequence end: no partial is read
    e_base = e_lo;
    const int* tlist = a.csr_t + (int64_t)bg * a.Tq * a.nslots;
    for (int i = tid; i < e_hi - e_lo; i += NT) s_tl[i] = tlist[e_lo + i];
    if (kStoreDs && a.ds) {
      const int* slist = a.csr_s + (int64_t)bg * a.Tq * a.nslots;
      for (int i = tid; i < e_hi - e_lo; i += NT) s_sl[i] = slist[e_lo + i];
    }
    __syncthreads();
  }

  // ---- this wave's 16 keys: K and V rows as B operands, kept in registers ----
  const int kw0 = key0 + wave * 16;
  const int mykey = kw0 + c16;
  uint4 kf[NKC], vf[NVC];
  {  // fragment-native copies: one coalesced 1 KB load per fragment
    const S* krf = reinterpret_cast<const S*>(a.krf) + (int64_t)bg * a.Tp * DK;
    const S* vrf = reinterpret_cast<const S*>(a.vrf) + (int64_t)bg * a.Tp * DV;
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc) kf[kc] = ld_rowfrag<T>(krf, kw0 >> 4, kc, DK, lane);
#pragma unroll
    for (int kc = 0; kc < NVC; ++kc) vf[kc] = ld_rowfrag<T>(vrf, kw0 >> 4, kc, DV, lane);
  }
  int mybe = 0x7fffffff, wave_be_min = 0x7fffffff, wave_be_max = 0x7fffffff;
  if (BR == kCompression) {
    mybe = s_be[wave * 16 + c16];
    wave_be_min = mybe;
    wave_be_max = mybe;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      wave_be_min = min(wave_be_min, __shfl_xor(wave_be_min, o));
      wave_be_max = max(wave_be_max, __shfl_xor(wave_be_max, o));
    }
  }

  // Wait for the K/V fragments here: otherwise the loop's first use of them becomes a
  // wait inside the loop body, which also stalls on the prefetch of the next chunk.
  __builtin_amdgcn_s_waitcnt(0);

  f32x4 dka[DK / 16], dva[DV / 16];
#pragma unroll
  for (int j = 0; j < DK / 16; ++j) dka[j] = zero4();
#pragma unroll
  for (int j = 0; j < DV / 16; ++j) dva[j] = zero4();

  const S* qbase = reinterpret_cast<const S*>(a.q) + b * a.sq_b;
  const S* obase = reinterpret_cast<const S*>(a.dout) + b * a.sdo_b;
  auto row_t = [&](int f) -> int {
    const int e = hdiv.div(f);
    return BR == kSelection ? s_tl[e - e_base] : e;
  };

  // ---- register prefetch of row chunks (pairs of adjacent rows): bf16 keeps two chunks
  // in flight (chunk c + 2 is requested into the registers chunk c was just staged from),
  // fp32 one ----
  struct Stage {
    uint4 pq[NQ][2], po[NO][2];
    int t;
    float4 st;  // lse2, delta, gate
  };
  // (the selection kernel at dk > 128 prefetches one chunk: two spill registers there)
  constexpr int kDepth = kTr && !(BR == kSelection && DK > 128) && DK > 64 ? 2 : 1;
  Stage stg0, stg1;
  stg0.t = stg1.t = -1;
  stg0.st = stg1.st = make_float4(INFINITY, 0.f, 1.f, 0.f);
  // Rows past the item's end re-read its last row (finite data); they are masked
  // (p = 0) through s_t = -1, so every load is unconditional and the loads of a chunk
  // issue back to back.
  const int sqh = (int)a.sq_h, sqt = (int)a.sq_t, soh = (int)a.sdo_h, sot = (int)a.sdo_t;
  auto load_row = [&](int f, const S* base, int sh, int st, int e) -> uint4 {
    const int fe = min(f, f_hi - 1);
    const int t = row_t(fe);
    const int h = grp * hpg + hdiv.mod(fe);
    return *reinterpret_cast<const uint4*>(base + e + ((int64_t)h * sh + (int64_t)t * st));
  };
  // the piece index c = tid + NT j is in range for every thread when the piece count
  // is a multiple of NT (known at compile time: no branch)
  auto in_q = [&](int c) { return QPCS % NT == 0 || c < QPCS; };
  auto in_o = [&](int c) { return OPCS % NT == 0 || c < OPCS; };
  auto load_chunk = [&](int fc, Stage& sg) __attribute__((always_inline)) {
    if constexpr (kTr) {
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        const int c = tid + NT * j;
        if (in_q(c)) sg.pq[j][0] = load_row(fc + c / (DK / EPF), qbase, sqh, sqt, (c % (DK / EPF)) * EPF);
      }
#pragma unroll
      for (int j = 0; j < NO; ++j) {
        const int c = tid + NT * j;
        if (in_o(c)) sg.po[j][0] = load_row(fc + c / (DV / EPF), obase, soh, sot, (c % (DV / EPF)) * EPF);
      }
    } else {
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      const int c = tid + NT * j;
      if (c < QPC) {
        const int rp = c % RPAIRS;
        const int e = (c / RPAIRS) * EPF;
        sg.pq[j][0] = load_row(fc + 2 * rp, qbase, sqh, sqt, e);
        sg.pq[j][1] = load_row(fc + 2 * rp + 1, qbase, sqh, sqt, e);
      }
    }
#pragma unroll
    for (int j = 0; j < NO; ++j) {
      const int c = tid + NT * j;
      if (c < OPC) {
        const int rp = c % RPAIRS;
        const int e = (c / RPAIRS) * EPF;
        sg.po[j][0] = load_row(fc + 2 * rp, obase, soh, sot, e);
        sg.po[j][1] = load_row(fc + 2 * rp + 1, obase, soh, sot, e);
      }
    }
    }
    if (tid < RC) {
      const int f = fc + tid;
      const int fe = min(f, f_hi - 1);
      const int t = row_t(fe);
      const int h = grp * hpg + hdiv.mod(fe);
      (void)h;
      // one 16-byte record per row; the heads of a timestep are adjacent
      sg.st = a.rstat[((int64_t)bg * a.Tq + t) * hpg + hdiv.mod(fe)];
      sg.t = f < f_hi ? t : -1;
    }
  };
  // position of chunk row r in the transposed (C-permuted for bf16) stage; rows 2k and
  // 2k+1 stay adjacent
  auto rowpos = [](int r) -> int { return sizeof(S) == 2 ? cperm_pos32(r) : r; };
  auto store_chunk = [&](int buf, const Stage& sg) __attribute__((always_inline)) {
    if constexpr (kTr) {
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        const int c = tid + NT * j;
        if (in_q(c))
          *reinterpret_cast<uint4*>(&Qs[buf][(c / (DK / EPF)) * QP + (c % (DK / EPF)) * EPF]) = sg.pq[j][0];
      }
#pragma unroll
      for (int j = 0; j < NO; ++j) {
        const int c = tid + NT * j;
        if (in_o(c))
          *reinterpret_cast<uint4*>(&Os[buf][(c / (DV / EPF)) * OP + (c % (DV / EPF)) * EPF]) = sg.po[j][0];
      }
    } else {
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      const int c = tid + NT * j;
      if (c < QPC) {
        const int rp = c % RPAIRS;
        const int e = (c / RPAIRS) * EPF;
        *reinterpret_cast<uint4*>(&Qs[buf][(2 * rp) * QP + e]) = sg.pq[j][0];
        *reinterpret_cast<uint4*>(&Qs[buf][(2 * rp + 1) * QP + e]) = sg.pq[j][1];
        PairT<S>::store(&QTs[buf][e * RP + rowpos(2 * rp)], RP, sg.pq[j][0], sg.pq[j][1]);
      }
    }
#pragma unroll
    for (int j = 0; j < NO; ++j) {
      const int c = tid + NT * j;
      if (c < OPC) {
        const int rp = c % RPAIRS;
        const int e = (c / RPAIRS) * EPF;
        *reinterpret_cast<uint4*>(&Os[buf][(2 * rp) * OP + e]) = sg.po[j][0];
        *reinterpret_cast<uint4*>(&Os[buf][(2 * rp + 1) * OP + e]) = sg.po[j][1];
        PairT<S>::store(&OTs[buf][e * RP + rowpos(2 * rp)], RP, sg.po[j][0], sg.po[j][1]);
      }
    }
    }
    if (tid < RC) {
      s_t[buf][tid] = sg.t;
      s_l2[buf][tid] = sg.st.x;
      s_dl[buf][tid] = sg.st.y;
      s_g[buf][tid] = sg.st.z;
    }
  };

  // stored dS of chunk cp (after a barrier that follows its tile writes): wave w stores
  // one 32-key fragment of one row subtile (selection: fragment w & 1 of subtile w >> 1;
  // otherwise fragment w & 3 of subtile w >> 2), lane (g4, c16) reading head c16 at the
  // 32-key chunk's keys 4 g4 + i and 16 + 4 g4 + i (its 8 slots) with two transpose loads
  auto flush_ds = [&](int cp) __attribute__((always_inline)) {
    if constexpr (kStoreDs && BR != kSelection) {
      const int rs = wave >> 2, kq = wave & 3;
      const int fr = f_lo + cp * RC + rs * 16;  // the subtile's rows: 16 heads of one timestep
      if (!a.ds || fr >= f_hi) return;           // wave-uniform
      const int t = hdiv.div(fr);
      const int hg = (fr - t * hpg) >> 4;
      const int kg = (key0 >> 5) + kq;  // the 32-key chunk
      int rel = kg;                     // its index among the timestep's stored chunks
      if (BR == kSliding) {             // chunks holding a key of (t - window, t]
        rel = kg - (max(0, t - a.window + 1) >> 5);
        if (rel < 0 || kg > (min(t, a.Tkv - 1) >> 5)) return;
      } else if (s_be[kq * 32] > t) {   // no key of the chunk visible (ascending block ends)
        return;
      }
      const uint4 v = ld_tr_pair(&s_dst[cp & 1][rs][(kq * 32 + 4 * g4 + (c16 >> 2)) * 16 + 4 * (c16 & 3)], 16 * 16);
      uint16_t* dsp = reinterpret_cast<uint16_t*>(a.ds) +
                      ((((int64_t)bg * a.Tq + t) * (hpg >> 4) + hg) * a.ds_nch + rel) * 512 + lane * 8;
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), reinterpret_cast<u32x4*>(dsp));
    }
    if constexpr (kStoreDs && BR == kSelection) {
      const int rs = wave >> 1, kc2 = wave & 1;
      const int fr = f_lo + cp * RC + rs * 16;  // the subtile's rows: 16 heads of one entry
      if (!a.ds || fr >= f_hi) return;           // wave-uniform
      const int e = hdiv.div(fr);
      const int hg = (fr - e * hpg) >> 4;
      const int t = s_tl[e - e_base], slot = s_sl[e - e_base];
      const uint4 v = ld_tr_pair(&s_dst[cp & 1][rs][(kc2 * 32 + 4 * g4 + (c16 >> 2)) * 16 + 4 * (c16 & 3)], 16 * 16);
      const int nhg = hpg >> 4, nsub = a.lprime >> 6;
      uint16_t* dsp = reinterpret_cast<uint16_t*>(a.ds) +
                      ((((int64_t)bg * a.Tq + t) * a.nslots + slot) * nsub + sub) * nhg * 1024 + hg * 1024 +
                      (kc2 * 64 + lane) * 8;
      // written once and read once by the dQ kernel: non-temporal
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), reinterpret_cast<u32x4*>(dsp));
    }
  };
  const int nchunks = (f_hi - f_lo + RC - 1) / RC;
  // One chunk: stage it from its registers, request the chunk kDepth further on into
  // them (bf16: unconditionally -- rows past the item's end re-read its last row and are
  // masked -- so that no load sits in a branch, whose join would make the compiler wait
  // for every load in flight), then the products.  A chunk wholly past the end (the
  // pair loop's padding) contributes nothing: its rows are masked.
  auto chunk = [&](int c, Stage& cur) __attribute__((always_inline)) {
    const int buf = c % NB;
    const int fc = f_lo + c * RC;
    if (NB == 1 && c > 0) __syncthreads();  // the previous chunk's reads are done
    store_chunk(buf, cur);
    if constexpr (kDepth == 2) load_chunk(fc + 2 * RC, cur);
    else if (c + 1 < nchunks) load_chunk(fc + RC, cur);
    __syncthreads();
    if (c > 0) flush_ds(c - 1);  // the previous chunk's dS tiles are complete

    // rows are in ascending t, so the chunk spans [t_min, t_max]
    const bool full = fc + RC <= f_hi;
    const int t_min = row_t(min(fc, f_hi - 1));
    const int t_max = row_t(min(fc + RC, f_hi) - 1);
    bool active, all_visible;
    if (BR == kSliding) {
      active = kw0 <= t_max && kw0 + 15 > t_min - a.window;
      all_visible = full && kw0 + 15 <= t_min && kw0 > t_max - a.window && kw0 + 15 < a.Tkv;
    } else if (BR == kCompression) {
      active = wave_be_min <= t_max;
      all_visible = full && wave_be_max <= t_min;
    } else {
      active = (!a.causal || kw0 <= t_max) && kw0 < blk_hi;
      all_visible = full && (!a.causal || kw0 + 15 <= t_min) && kw0 + 15 < blk_hi;
    }

    // Waves whose keys no row of the chunk can see still run the (fully masked) products:
    // a branch around them makes the compiler shuttle the dK/dV accumulators between
    // register files on every chunk, which costs more than the skipped work.
    (void)active;
    {
      f32x4 pt[RC / 16], dst[RC / 16];
#pragma unroll
      for (int rs = 0; rs < RC / 16; ++rs) {
        f32x4 sacc = zero4(), pacc = zero4();
        const S* qrow = &Qs[buf][(rs * 16 + c16) * QP];
        const S* orow = &Os[buf][(rs * 16 + c16) * OP];
#pragma unroll
        for (int kc = 0; kc < NKC; ++kc) sacc = Mma<T>::run(sacc, frag_std<T>(qrow + kc * KC, g4), kf[kc]);
#pragma unroll
        for (int kc = 0; kc < NVC; ++kc) pacc = Mma<T>::run(pacc, frag_std<T>(orow + kc * KC, g4), vf[kc]);
        // the lane's four rows rs*16 + 4*g4 + i: their statistics as one 16-byte read each,
        // the mask applied to the exponent argument (no divergent branch)
        const int r4 = rs * 16 + 4 * g4;
        const float4 l2v = *reinterpret_cast<const float4*>(&s_l2[buf][r4]);
        const float4 dlv = *reinterpret_cast<const float4*>(&s_dl[buf][r4]);
        const float4 gv = *reinterpret_cast<const float4*>(&s_g[buf][r4]);
        const int4 tv = *reinterpret_cast<const int4*>(&s_t[buf][r4]);
        const float l2a[4] = {l2v.x, l2v.y, l2v.z, l2v.w}, dla[4] = {dlv.x, dlv.y, dlv.z, dlv.w};
        const float ga[4] = {gv.x, gv.y, gv.z, gv.w};
        const int ta[4] = {tv.x, tv.y, tv.z, tv.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // masked elements: the argument clamped to -inf by a min with a selected
          // constant, the conditions combined with bitwise operators (a select of the
          // argument itself, or short-circuit ands, become divergent branches in the
          // loop); chunks whose rows all see the wave's keys skip the mask (uniform)
          // (compression keeps the select: measured faster there)
          float arg = sacc[i] * scale2 - l2a[i];
          if (BR == kCompression) {
            arg = (all_visible || (ta[i] >= 0 && mybe <= ta[i])) ? arg : -INFINITY;
          } else if (!all_visible) {
            const int t = ta[i];
            bool vis;
            if (BR == kSliding) vis = (t >= 0) & (mykey <= t) & (mykey > t - a.window) & (mykey < a.Tkv);
            else vis = (t >= 0) & ((a.causal == 0) | (mykey <= t)) & (mykey < blk_hi);
            arg = fminf(arg, vis ? INFINITY : -INFINITY);
          }
          // lse2 is +inf for rows that saw no key: p = 0 there
          const float p = fast_exp2(arg) * ga[i];  // gated: g dO
          pt[rs][i] = p;
          dst[rs][i] = p * (pacc[i] - dla[i]);
        }
        if constexpr (kStoreDs) {  // the lane's four heads of its key, into the chunk's tile
          if (a.ds)
            *reinterpret_cast<uint2*>(&s_dst[c & 1][rs][(wave * 16 + c16) * 16 + 4 * g4]) =
                make_uint2(pack_bf16x2(dst[rs][0], dst[rs][1]), pack_bf16x2(dst[rs][2], dst[rs][3]));
        }
      }
#pragma unroll
      for (int kc2 = 0; kc2 < RC / CK; ++kc2) {
        const uint4 pf = CFrag<T>::pack(pt[kc2 * CT], pt[kc2 * CT + CT - 1]);
        const uint4 sf = CFrag<T>::pack(dst[kc2 * CT], dst[kc2 * CT + CT - 1]);
        if constexpr (kTr) {
          // A = dO^T / Q^T (16 features x the 32 rows of the C-permuted CFrag order):
          // lanes 4*rho+q of group g4 address row kc2*32 + 4*g4 + rho (then +16),
          // features 4q..4q+3 of the 16-feature tile
          const int r0 = kc2 * CK + 4 * g4 + (c16 >> 2);
          const int f4 = 4 * (c16 & 3);
#pragma unroll
          for (int j = 0; j < DV / 16; ++j)
            dva[j] = Mma<T>::run(dva[j], ld_tr_pair(&Os[buf][r0 * OP + j * 16 + f4], 16 * OP), pf);
#pragma unroll
          for (int j = 0; j < DK / 16; ++j)
            dka[j] = Mma<T>::run(dka[j], ld_tr_pair(&Qs[buf][r0 * QP + j * 16 + f4], 16 * QP), sf);
        } else {
#pragma unroll
        for (int j = 0; j < DV / 16; ++j)
          dva[j] = Mma<T>::run(dva[j], frag_cperm<T>(&OTs[buf][(j * 16 + c16) * RP + kc2 * CK], g4), pf);
#pragma unroll
        for (int j = 0; j < DK / 16; ++j)
          dka[j] = Mma<T>::run(dka[j], frag_cperm<T>(&QTs[buf][(j * 16 + c16) * RP + kc2 * CK], g4), sf);
        }
      }
    }
  };
  if constexpr (kDepth == 2) {
    if (nchunks > 0) {
      load_chunk(f_lo, stg0);
      load_chunk(f_lo + RC, stg1);
    }
    int c = 0;
    for (; c < nchunks; c += 2) {  // an odd count runs one padding chunk
      chunk(c, stg0);
      chunk(c + 1, stg1);
    }
    if (kStoreDs && a.ds && c > 0) {
      __syncthreads();
      flush_ds(c - 1);
    }
  } else {
    if (nchunks > 0) load_chunk(f_lo, stg0);
    for (int c = 0; c < nchunks; ++c) chunk(c, stg0);
    if (kStoreDs && a.ds && nchunks > 0) {  // the last chunk's dS tiles
      __syncthreads();
      flush_ds(nchunks - 1);
    }
  }

  // ---- direct mode: add this item's dK / dV into the caller's, or store them (lane holds
  // dK^T[d = 16j + 4*g4 + i][key = mykey]: four consecutive features of one key) ----
  if (a.direct) {
    if (mykey >= a.Tkv) return;
    S* kp = reinterpret_cast<S*>(a.dk) + b * a.sdk_b + grp * a.sdk_g + (int64_t)mykey * a.sdk_t;
    S* vp = reinterpret_cast<S*>(a.dv) + b * a.sdv_b + grp * a.sdv_g + (int64_t)mykey * a.sdv_t;
    if (a.dkdv_ow) {  // the item owns its keys: store instead of read-modify-write
#pragma unroll
      for (int j = 0; j < DK / 16; ++j) set4<T>(kp, (int64_t)(j * 16 + 4 * g4), a.sdk_d, dka[j] * a.scale);
#pragma unroll
      for (int j = 0; j < DV / 16; ++j) set4<T>(vp, (int64_t)(j * 16 + 4 * g4), a.sdv_d, dva[j]);
      return;
    }
#pragma unroll
    for (int j = 0; j < DK / 16; ++j) add4<T>(kp, (int64_t)(j * 16 + 4 * g4), a.sdk_d, dka[j] * a.scale);
#pragma unroll
    for (int j = 0; j < DV / 16; ++j) add4<T>(vp, (int64_t)(j * 16 + 4 * g4), a.sdv_d, dva[j]);
    return;
  }
  // ---- write this item's partial (in the element type: the reduce sums the items' partials
  // in fp32): lane holds dK^T[d = 16j + 4*g4 + i][key = mykey] ----
  S* pp = reinterpret_cast<S*>(a.partial) + ((int64_t)bg * a.items_per_bg + item) * KEYS * (DK + DV) +
          (int64_t)(wave * 16 + c16) * (DK + DV);
#pragma unroll
  for (int j = 0; j < DK / 16; ++j) store4<T>(pp + j * 16 + 4 * g4, dka[j] * a.scale);
#pragma unroll
  for (int j = 0; j < DV / 16; ++j) store4<T>(pp + DK + j * 16 + 4 * g4, dva[j]);
}

template <typename T, int DK, int DV, int BR>
void launch_attn_bwd_dkdv(const AttnArgs& a, hipStream_t s) {
  if (a.items_per_bg <= 0) return;
  dim3 grid(a.items_per_bg, a.B * a.G);
  hipLaunchKernelGGL((attn_bwd_dkdv_kernel<T, DK, DV, BR>), grid, dim3(4 * dkdv_keys(BR)), 0, s, a);
}

}  // namespace nsa
