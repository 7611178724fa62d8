// C ABI entry points (declared in include/nsa_hip.h): argument validation, the
// workspace layout, and the launch sequence of each NSA attention operator.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "../../include/nsa_hip.h"
#include "nsa_attn.h"
#include "nsa_attn_bwd_dkdv.h"
#include "nsa_kernels.h"

using namespace nsa;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_hip(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NSA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return NSA_OK;
}

bool dims_supported(int dk, int dv) {
#define NSA_SUP(A, B) \
  if (dk == A && dv == B) return true;
  NSA_HEAD_DIMS(NSA_SUP)
#undef NSA_SUP
  return false;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct Shape {
  int br, dtype, Z, H, G, Tq, Tkv, dk, dv, nslots, lprime;
  int window = 0;
  int q0 = 0;  // absolute position of query row 0 (forward extensions)
  int hpg() const { return H / G; }
  int Tp() const { return ((Tkv + 63) / 64) * 64 + 64; }
  int esz() const { return dtype == NSA_F32 ? 4 : 2; }
  int nblk() const { return br == kSelection ? (Tkv + lprime - 1) / lprime : 0; }
  int nsubblk() const { return (lprime + 63) / 64; }
  // dK/dV work items per (b, g): key tiles x query segments of sg entries
  int items_for(int sg) const {
    if (br == kSelection) return nsubblk() * (nblk() + (int)(((int64_t)Tq * nslots + sg - 1) / sg));
    return ((Tkv + dkdv_keys(br) - 1) / dkdv_keys(br)) * dkdv_nseg(br, Tq, window, sg);
  }
  // sliding window with at least one 128-key tile per CU: a work item owns a key tile
  // with all its query rows and accumulates into dK / dV itself (no partials, no
  // reduce pass)
  bool direct() const {
    return br == kSliding && (int64_t)Z * G * ((Tkv + dkdv_keys(br) - 1) / dkdv_keys(br)) >= kDkdvDirectItems;
  }
  // segment length: the whole query span in direct mode; 256 entries when that leaves
  // 4096 work items or more; else the multiple of 32 in [128, 256] that needs the
  // fewest entry-steps per CU, ceil(items / 256 CUs) x segment (ties to the shorter),
  // so that a small launch does not end on a partly filled round of work items
  int seg() const {
    if (direct()) return min(window + dkdv_keys(br) - 1, Tq + dkdv_keys(br) - 1);
    if ((int64_t)Z * G * items_for(kSegTMax) >= 4096) return kSegTMax;
    int best = kSegTMax / 2;
    int64_t best_cost = INT64_MAX;
    for (int sg = kSegTMax / 2; sg <= kSegTMax; sg += 32) {
      const int64_t cost = ((int64_t)Z * G * items_for(sg) + 255) / 256 * sg;
      if (cost < best_cost) best = sg, best_cost = cost;
    }
    return best;
  }
  int items_per_bg() const { return items_for(seg()); }
  // selection backward with stored dS (bf16, whole 16-head groups, 64-key sub-blocks):
  // the dK/dV kernel runs first and stores dS, the dQ kernel reads it
  // (selection); sliding window / compression: bf16, whole 16-head groups, dS stored per
  // (timestep, 32-key chunk it sees)
  // The stored dS grows with the batch and the window / compressed length / slot count
  // (about 2 bytes per visible (query row, key) pair): beyond kMaxStoredDs every branch
  // recomputes dS in its dQ kernel instead.
  static constexpr size_t kMaxStoredDs = size_t(6) << 30;
  bool stored_ds() const {
    if (dtype != NSA_BF16 || hpg() % 16) return false;
    if (br == kSelection) return lprime % 64 == 0 && nslots > 0 && sel_ds_bytes() <= kMaxStoredDs;
    // compression: the dQ pass keeps each 32-key chunk's first block end in LDS
    if (br == kCompression && (Tkv + 31) / 32 > kDqCbeMax) return false;
    return dense_ds_bytes() <= kMaxStoredDs;
  }
  size_t sel_ds_bytes() const { return (size_t)Z * H * Tq * nslots * lprime * 2; }
  size_t dense_ds_bytes() const { return (size_t)Z * G * Tq * (hpg() / 16) * ds_nch() * 1024; }
  // dense: 32-key chunks stored per (timestep, head group)
  int ds_nch() const {
    const int all = (Tkv + 31) / 32;
    return br == kSliding ? min((window + 62) / 32, all + 1) : all;
  }
  size_t ds_bytes() const {
    if (!stored_ds()) return 0;
    if (br == kSelection) return sel_ds_bytes();
    return dense_ds_bytes();
  }
};

struct Layout {
  size_t krf = 0, kcf = 0, vrf = 0, vcf = 0, rstat = 0, clean = 0, chunk = 0, csr_off = 0, csr_t = 0,
         seg_off = 0, csr_s = 0, ds = 0, partial = 0, total = 0;
};

// Offsets into the caller's workspace (every buffer 256-byte aligned).
Layout make_layout(const Shape& s, bool bwd) {
  Layout L;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t at = off;
    off += align256(bytes);
    return at;
  };
  const size_t BG = (size_t)s.Z * s.G;
  const size_t kbytes = BG * s.Tp() * s.dk * s.esz();
  const size_t vbytes = BG * s.Tp() * s.dv * s.esz();
  // fragment-native operands (every MFMA fragment one contiguous 1 KB run)
  L.krf = take(kbytes);
  if (bwd) {
    L.kcf = take(kbytes);
    L.vrf = take(vbytes);
  } else {
    L.vcf = take(vbytes);
  }
  if (bwd) {
    L.rstat = take((size_t)s.Z * s.H * s.Tq * 16);
  }
  if (s.br == kSelection) {
    L.clean = take(BG * s.Tq * s.nslots * 4);
    if (bwd) {
      L.chunk = take(BG * sel_csr_chunks(s.Tq) * s.nblk() * 4);
      L.csr_off = take(BG * (s.nblk() + 1) * 4);
      L.seg_off = take(BG * (s.nblk() + 1) * 4);
      L.csr_t = take(BG * s.Tq * s.nslots * 4);
      if (s.stored_ds()) {
        L.csr_s = take(BG * s.Tq * s.nslots * 4);
        L.ds = take(s.ds_bytes());
      }
    }
  }
  if (bwd && s.br != kSelection && s.stored_ds()) L.ds = take(s.ds_bytes());
  if (bwd && !s.direct()) L.partial = take(BG * s.items_per_bg() * dkdv_keys(s.br) * (size_t)(s.dk + s.dv) * s.esz());
  L.total = off;
  return L;
}

// Unit feature stride and 16-byte aligned rows; the strides of size-1 axes are
// never used to address memory, so they are not checked.  The head and time strides
// must fit 32 bits (the kernels multiply them as 32-bit operands into 64-bit offsets).
bool row_ok(const void* p, int64_t inner, int64_t s0, int64_t s1, int64_t s2, int esz, int n0 = 2, int n1 = 2,
            int n2 = 2) {
  if (inner != 1) return false;
  if (((uintptr_t)p) % 16) return false;
  if ((n1 != 1 && (s1 < 0 || s1 > INT32_MAX)) || (n2 != 1 && (s2 < 0 || s2 > INT32_MAX))) return false;
  return (n0 == 1 || (s0 * esz) % 16 == 0) && (n1 == 1 || (s1 * esz) % 16 == 0) && (n2 == 1 || (s2 * esz) % 16 == 0);
}

int validate(const Shape& s) {
  if (s.dtype != NSA_F32 && s.dtype != NSA_BF16) return fail(NSA_ERR_INVALID, "dtype %d not supported", s.dtype);
  if (s.q0 < 0) return fail(NSA_ERR_INVALID, "q_offset=%d must be >= 0", s.q0);
  if (s.Z <= 0 || s.H <= 0 || s.G <= 0 || s.Tq < 0 || s.Tkv < 0)
    return fail(NSA_ERR_INVALID, "bad shape Z=%d H=%d G=%d Tq=%d Tkv=%d", s.Z, s.H, s.G, s.Tq, s.Tkv);
  if (s.H % s.G) return fail(NSA_ERR_INVALID, "H=%d not a multiple of n_kv_groups=%d", s.H, s.G);
  if (!dims_supported(s.dk, s.dv))
    return fail(NSA_ERR_UNSUPPORTED, "no kernel for head dims dk=%d dv=%d", s.dk, s.dv);
  if (s.br == kSelection) {
    if (s.lprime <= 0 || s.lprime % 16) return fail(NSA_ERR_INVALID, "block_size_selection=%d must be a positive multiple of 16", s.lprime);
    if (s.nslots < 0 || s.nslots > 64) return fail(NSA_ERR_INVALID, "n_slots=%d outside [0, 64]", s.nslots);
    if (s.nblk() > kSelMaxBlocks) return fail(NSA_ERR_UNSUPPORTED, "%d selection blocks exceed %d", s.nblk(), kSelMaxBlocks);
  }
  return NSA_OK;
}

AttnArgs base_args(const Shape& s, float scale) {
  AttnArgs a;
  memset(&a, 0, sizeof(a));
  a.B = s.Z;
  a.H = s.H;
  a.G = s.G;
  a.hpg = s.hpg();
  a.Tq = s.Tq;
  a.Tkv = s.Tkv;
  a.Tp = s.Tp();
  a.q0 = s.q0;
  a.scale = scale;
  a.lprime = s.lprime > 0 ? s.lprime : 1;
  a.nslots = s.nslots;
  a.nblk = s.nblk();
  a.causal = 1;
  return a;
}

template <typename P> P* at(void* ws, size_t off) { return reinterpret_cast<P*>(reinterpret_cast<char*>(ws) + off); }

struct FwdIO {
  const void *Q, *K, *V;
  void* Out;
  float *L, *M;
  int64_t sq[4], sk[4], sv[4], so[4], sl[3], sm[3];
  // sliding extension only: gated mix epilogue (null mix_out: none)
  const void* mix_o0 = nullptr;
  const void* mix_o1 = nullptr;
  const float* mix_gates = nullptr;
  void* mix_out = nullptr;
  int64_t sx[3] = {0, 0, 0};
};

int run_fwd(const Shape& s, const FwdIO& io, float scale, int window, const int32_t* block_ends, const void* idx,
            const int64_t* sidx, int idx64, int fallback, int causal, void* ws, size_t ws_bytes, hipStream_t st) {
  int rc = validate(s);
  if (rc) return rc;
  if (!row_ok(io.Q, io.sq[3], io.sq[0], io.sq[1], io.sq[2], s.esz(), s.Z, s.H, s.Tq))
    return fail(NSA_ERR_LAYOUT, "Q needs unit feature stride and 16-byte aligned rows");
  if (!row_ok(io.Out, io.so[3], io.so[0], io.so[1], io.so[2], s.esz(), s.Z, s.H, s.Tq))
    return fail(NSA_ERR_LAYOUT, "Out needs unit feature stride and 16-byte aligned rows");
  if (s.br == kSliding && window <= 0) return fail(NSA_ERR_INVALID, "window_size=%d must be positive", window);
  if (io.mix_out) {
    if (!io.mix_o0 || !io.mix_o1 || !io.mix_gates) return fail(NSA_ERR_INVALID, "mix needs mix_o0, mix_o1 and mix_gates");
    if (!row_ok(io.mix_out, 1, io.sx[0], io.sx[1], io.sx[2], s.esz(), s.Z, s.H, s.Tq) ||
        !row_ok(io.mix_o0, io.so[3], io.so[0], io.so[1], io.so[2], s.esz(), s.Z, s.H, s.Tq) ||
        !row_ok(io.mix_o1, io.so[3], io.so[0], io.so[1], io.so[2], s.esz(), s.Z, s.H, s.Tq))
      return fail(NSA_ERR_LAYOUT, "mix outputs need 16-byte aligned unit-stride rows");
  }
  const Layout L = make_layout(s, false);
  if (ws_bytes < L.total) return fail(NSA_ERR_WORKSPACE, "workspace %zu bytes < required %zu", ws_bytes, L.total);
  if (s.Tq == 0) return NSA_OK;

  AttnArgs a = base_args(s, scale);
  a.q = io.Q;
  a.sq_b = io.sq[0];
  a.sq_h = io.sq[1];
  a.sq_t = io.sq[2];
  a.o = io.Out;
  a.so_b = io.so[0];
  a.so_h = io.so[1];
  a.so_t = io.so[2];
  a.L = io.L;
  a.sl_b = io.sl[0];
  a.sl_h = io.sl[1];
  a.sl_t = io.sl[2];
  a.M = io.M;
  a.sm_b = io.sm[0];
  a.sm_h = io.sm[1];
  a.sm_t = io.sm[2];
  a.window = window;
  a.block_ends = block_ends;
  a.causal = causal;
  a.mix_out = io.mix_out;
  a.smx_b = io.sx[0];
  a.smx_h = io.sx[1];
  a.smx_t = io.sx[2];
  a.mix_o0 = io.mix_o0;
  a.mix_o1 = io.mix_o1;
  a.mix_gates = io.mix_gates;
  a.krf = at<char>(ws, L.krf);
  a.vcf = at<char>(ws, L.vcf);

  launch_repack_kv(s.dtype, io.K, io.sk, s.dk, const_cast<void*>(a.krf), nullptr, io.V, io.sv, s.dv, nullptr,
                   const_cast<void*>(a.vcf), s.Z, s.G, s.Tkv, a.Tp, st);
  if (s.br == kSelection) {
    launch_sel_clean(idx, idx64, sidx[0], sidx[1], sidx[2], sidx[3], s.Z, s.G, s.Tq, s.nslots, s.nslots, s.lprime,
                     s.Tkv, fallback, causal, at<int>(ws, L.clean), nullptr, s.nblk(), s.q0, st);
    a.sel = at<int>(ws, L.clean);
  }
  if ((rc = check_hip("prep"))) return rc;
  {
    TimingScope ts(kIdFwd + s.br, st);
    if (!dispatch_attn_fwd(s.dtype, s.dk, s.dv, s.br, a, st)) return fail(NSA_ERR_UNSUPPORTED, "no forward kernel");
  }
  return check_hip("attention forward");
}

struct BwdIO {
  const void *Q, *K, *V, *Out, *dOut;
  const float *L, *M;
  void *dQ, *dK, *dV;
  int64_t sq[4], sk[4], sv[4], so[4], sl[3], sm[3], sdq[4], sdk[4], sdv[4];
  int dq_acc = 0;                   // extension entry points only: add into dQ
  int dkdv_ow = 0;                  // extension entry points only: overwrite dK / dV
  const float* delta_in = nullptr;  // extension entry points only: precomputed row sums
  const float* row_gate = nullptr;  // extension entry points only: per-row gate of dOut
  float* row_dot = nullptr;         // extension entry points only: receives sum_d dOut * Out
  int defer_dq = 0;                 // extension entry points only: everything but the dQ kernel
  // nsa_sliding_window_bwd_pair only: a deferred compression backward's workspace, whose
  // dQ the sliding-window dQ kernel adds in the same pass
  const void* pair_ws = nullptr;
  size_t pair_ws_bytes = 0;
  const int32_t* pair_block_ends = nullptr;
  int pair_n_blocks = 0;
};

int set_bwd_ext(BwdIO& io, int flags, const float* delta_in, const float* row_gate, float* row_dot) {
  if (flags & ~(NSA_BWD_DQ_ACCUMULATE | NSA_BWD_DKDV_OVERWRITE | NSA_BWD_DQ_DEFER))
    return fail(NSA_ERR_INVALID, "bwd_flags=%d has unknown bits", flags);
  io.dq_acc = (flags & NSA_BWD_DQ_ACCUMULATE) ? 1 : 0;
  io.dkdv_ow = (flags & NSA_BWD_DKDV_OVERWRITE) ? 1 : 0;
  io.defer_dq = (flags & NSA_BWD_DQ_DEFER) ? 1 : 0;
  io.delta_in = delta_in;
  io.row_gate = row_gate;
  io.row_dot = row_dot;
  return NSA_OK;
}

int run_bwd(const Shape& s, const BwdIO& io, float scale, int window, const int32_t* block_ends, const void* idx,
            const int64_t* sidx, int idx64, int fallback, int causal, void* ws, size_t ws_bytes, hipStream_t st) {
  int rc = validate(s);
  if (rc) return rc;
  if (!row_ok(io.Q, io.sq[3], io.sq[0], io.sq[1], io.sq[2], s.esz(), s.Z, s.H, s.Tq))
    return fail(NSA_ERR_LAYOUT, "Q needs unit feature stride and 16-byte aligned rows");
  if (!row_ok(io.dOut, io.so[3], io.so[0], io.so[1], io.so[2], s.esz(), s.Z, s.H, s.Tq))
    return fail(NSA_ERR_LAYOUT, "dOut (Out strides) needs unit feature stride and 16-byte aligned rows");
  if (!row_ok(io.dQ, io.sdq[3], io.sdq[0], io.sdq[1], io.sdq[2], s.esz(), s.Z, s.H, s.Tq))
    return fail(NSA_ERR_LAYOUT, "dQ needs unit feature stride and 16-byte aligned rows");
  if (s.br == kSliding && window <= 0) return fail(NSA_ERR_INVALID, "window_size=%d must be positive", window);
  if (io.row_dot && io.delta_in) return fail(NSA_ERR_INVALID, "row_dot needs delta_in = null (it is computed from Out)");
  const Layout L = make_layout(s, true);
  if (ws_bytes < L.total) return fail(NSA_ERR_WORKSPACE, "workspace %zu bytes < required %zu", ws_bytes, L.total);
  if (io.defer_dq && !s.stored_ds())
    return fail(NSA_ERR_INVALID, "NSA_BWD_DQ_DEFER needs a backward that stores dS (nsa_bwd_dq_deferrable)");

  AttnArgs a = base_args(s, scale);
  if (io.pair_ws) {
    // the deferred compression backward over the same queries: its workspace layout
    const Shape sc{kCompression, s.dtype, s.Z, s.H, s.G, s.Tq, io.pair_n_blocks, s.dk, s.dv, 0, 64};
    if (s.br != kSliding || !s.stored_ds() || !sc.stored_ds())
      return fail(NSA_ERR_INVALID, "the paired dQ needs both backwards to store dS (nsa_bwd_dq_deferrable)");
    if (io.pair_n_blocks < 0 || (io.pair_n_blocks > 0 && !io.pair_block_ends))
      return fail(NSA_ERR_INVALID, "compression block ends are null or n_blocks=%d is negative", io.pair_n_blocks);
    const Layout Lc = make_layout(sc, true);
    if (io.pair_ws_bytes < Lc.total)
      return fail(NSA_ERR_WORKSPACE, "compression workspace %zu bytes < required %zu", io.pair_ws_bytes, Lc.total);
    void* wc = const_cast<void*>(io.pair_ws);
    a.pair_kcf = at<char>(wc, Lc.kcf);
    a.pair_ds = at<char>(wc, Lc.ds);
    a.pair_block_ends = io.pair_block_ends;
    a.pair_Tkv = io.pair_n_blocks;
    a.pair_Tp = sc.Tp();
    a.pair_ds_nch = sc.ds_nch();
  }
  a.dk = io.dK;
  a.sdk_b = io.sdk[0];
  a.sdk_g = io.sdk[1];
  a.sdk_t = io.sdk[2];
  a.sdk_d = io.sdk[3];
  a.dv = io.dV;
  a.sdv_b = io.sdv[0];
  a.sdv_g = io.sdv[1];
  a.sdv_t = io.sdv[2];
  a.sdv_d = io.sdv[3];
  a.dkdv_ow = io.dkdv_ow;
  if (s.Tq == 0) {  // no query rows: dK / dV receive nothing (zeros when overwritten)
    if (!io.dkdv_ow) return NSA_OK;
    launch_zero_dkdv(s.dtype, s.dk, s.dv, a, st);
    return check_hip("dK/dV zero fill");
  }
  a.q = io.Q;
  a.sq_b = io.sq[0];
  a.sq_h = io.sq[1];
  a.sq_t = io.sq[2];
  // the reference reads dOut with Out's strides (nsa/kernels.py:1378-1384)
  a.o = const_cast<void*>(io.Out);
  a.so_b = io.so[0];
  a.so_h = io.so[1];
  a.so_t = io.so[2];
  a.dout = io.dOut;
  a.sdo_b = io.so[0];
  a.sdo_h = io.so[1];
  a.sdo_t = io.so[2];
  a.L = const_cast<float*>(io.L);
  a.sl_b = io.sl[0];
  a.sl_h = io.sl[1];
  a.sl_t = io.sl[2];
  a.M = const_cast<float*>(io.M);
  a.sm_b = io.sm[0];
  a.sm_h = io.sm[1];
  a.sm_t = io.sm[2];
  a.dq = io.dQ;
  a.sdq_b = io.sdq[0];
  a.sdq_h = io.sdq[1];
  a.sdq_t = io.sdq[2];
  a.dq_acc = io.dq_acc;
  a.delta_in = io.delta_in;
  a.row_gate = io.row_gate;
  a.row_dot = io.row_dot;
  a.window = window;
  a.block_ends = block_ends;
  a.causal = causal;
  const bool sel = s.br == kSelection;
  auto opt = [&](size_t off, bool use) -> void* { return use ? at<char>(ws, off) : nullptr; };
  a.krf = at<char>(ws, L.krf);
  a.kcf = at<char>(ws, L.kcf);
  a.vrf = at<char>(ws, L.vrf);
  a.rstat = at<float4>(ws, L.rstat);
  a.items_per_bg = s.items_per_bg();
  a.seg = s.seg();
  a.direct = s.direct() ? 1 : 0;
  a.partial = at<char>(ws, L.partial);

  launch_repack_kv(s.dtype, io.K, io.sk, s.dk, const_cast<void*>(a.krf), const_cast<void*>(a.kcf), io.V, io.sv,
                   s.dv, const_cast<void*>(a.vrf), nullptr, s.Z, s.G, s.Tkv, a.Tp, st);
  if (s.br == kSelection) {
    launch_sel_clean(idx, idx64, sidx[0], sidx[1], sidx[2], sidx[3], s.Z, s.G, s.Tq, s.nslots, s.nslots, s.lprime,
                     s.Tkv, fallback, causal, at<int>(ws, L.clean), at<int>(ws, L.chunk), s.nblk(), 0, st);
    launch_sel_csr(at<int>(ws, L.clean), at<int>(ws, L.chunk), s.Z, s.G, s.Tq, s.nslots, s.nblk(),
                   at<int>(ws, L.csr_off), at<int>(ws, L.csr_t), s.stored_ds() ? at<int>(ws, L.csr_s) : nullptr,
                   at<int>(ws, L.seg_off), s.seg(), st);
    a.sel = at<int>(ws, L.clean);
    a.csr_off = at<int>(ws, L.csr_off);
    a.csr_t = at<int>(ws, L.csr_t);
    a.seg_off = at<int>(ws, L.seg_off);
  }
  if ((rc = check_hip("backward prep"))) return rc;
  auto dq = [&]() -> int {
    {
      TimingScope ts(kIdDq + s.br, st);
      if (!dispatch_attn_bwd_dq(s.dtype, s.dk, s.dv, s.br, a, st)) return fail(NSA_ERR_UNSUPPORTED, "no dQ kernel");
    }
    return check_hip("dQ kernel");
  };
  // stored dS: the row statistics first, then dK/dV (which stores dS), then dQ from it;
  // otherwise the dQ kernel computes the statistics and dK/dV follows
  if (s.stored_ds()) {
    if (s.br == kSelection) a.csr_s = at<int>(ws, L.csr_s);
    a.ds = at<char>(ws, L.ds);
    a.ds_nch = s.ds_nch();
    {
      TimingScope ts(kIdPrep, st);
      if (!launch_row_stats(s.dtype, s.dv, a, st)) return fail(NSA_ERR_UNSUPPORTED, "no row statistics kernel");
    }
    if ((rc = check_hip("row statistics"))) return rc;
  } else if ((rc = dq())) {
    return rc;
  }
  {
    TimingScope ts(kIdDkdv + s.br, st);
    if (!dispatch_attn_bwd_dkdv(s.dtype, s.dk, s.dv, s.br, a, st)) return fail(NSA_ERR_UNSUPPORTED, "no dK/dV kernel");
  }
  if ((rc = check_hip("dK/dV kernel"))) return rc;
  {
    TimingScope ts(kIdReduce, st);
    if (!a.direct) launch_partial_reduce(s.dtype, s.dk, s.dv, s.br, a, st);
  }
  if ((rc = check_hip("dK/dV reduce"))) return rc;
  if (s.stored_ds() && !io.defer_dq && (rc = dq())) return rc;
  return NSA_OK;
}

// Scratch memory of the allocation-free entry point (nsa_sliding_window_fwd_noalloc):
// a fixed device array that every GPU the library runs on holds until the process ends.
// Host code never uses the array's name as an address: each device's copy is looked up
// once with hipGetSymbolAddress and that pointer is passed to the kernels.
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// This device's copy of `scratch` (looked up on the first call per device, with that
// device current).
int scratch_ptr(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(NSA_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(NSA_ERR_UNSUPPORTED, "device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return fail(NSA_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return NSA_OK;
}

}  // namespace

int nsa::set_error(int code, const char* msg) { return fail(code, "%s", msg); }

extern "C" {

int nsa_abi_version(void) { return 5; }
const char* nsa_last_error(void) { return g_err; }
int nsa_head_dims_supported(int dtype, int dk, int dv) {
  return (dtype == NSA_F32 || dtype == NSA_BF16) && dims_supported(dk, dv);
}

size_t nsa_fwd_workspace_size(int branch, int dtype, int Z, int H, int G, int Tq, int Tkv, int dk, int dv, int nslots,
                              int lprime) {
  Shape s{branch, dtype, Z, H, G, Tq, Tkv, dk, dv, nslots, lprime > 0 ? lprime : 64};
  if (G <= 0 || H % G) return 0;
  return make_layout(s, false).total;
}
size_t nsa_bwd_workspace_size(int branch, int dtype, int Z, int H, int G, int Tq, int Tkv, int dk, int dv, int nslots,
                              int lprime, int window_size) {
  Shape s{branch, dtype, Z, H, G, Tq, Tkv, dk, dv, nslots, lprime > 0 ? lprime : 64, window_size > 0 ? window_size : 1};
  if (G <= 0 || H % G) return 0;
  return make_layout(s, true).total;
}

int nsa_bwd_dq_deferrable(int branch, int dtype, int Z, int H, int G, int Tq, int Tkv, int dk, int dv, int nslots,
                          int lprime, int window_size) {
  Shape s{branch, dtype, Z, H, G, Tq, Tkv, dk, dv, nslots, lprime > 0 ? lprime : 64, window_size > 0 ? window_size : 1};
  if (G <= 0 || H % G || Z < 0 || Tq < 0) return 0;
  return s.stored_ds() ? 1 : 0;
}

int nsa_bwd_dkdv_plan(int branch, int Z, int H, int G, int Tq, int Tkv, int nslots, int lprime, int window_size,
                      int* items_per_bg, int* segment) {
  Shape s{branch, NSA_BF16, Z, H, G, Tq, Tkv, 64, 64, nslots, lprime > 0 ? lprime : 64, window_size > 0 ? window_size : 1};
  if (Z <= 0 || G <= 0 || H % G || Tq < 0 || Tkv < 0) return fail(NSA_ERR_INVALID, "bad shape");
  if (items_per_bg) *items_per_bg = s.items_per_bg();
  if (segment) *segment = s.seg();
  return NSA_OK;
}

#define NSA_FWD_IO                                                                                    \
  FwdIO io{Q, K, V, Out, L, M,                                                                        \
           {stride_qz, stride_qh, stride_qm, stride_qk}, {stride_kz, stride_kg, stride_kn, stride_kk}, \
           {stride_vz, stride_vg, stride_vn, stride_vk}, {stride_oz, stride_oh, stride_om, stride_ok}, \
           {stride_lz, stride_lh, stride_lm}, {stride_mz, stride_mh, stride_mm}};
#define NSA_BWD_IO                                                                                        \
  BwdIO io{Q, K, V, Out, dOut, L, M, dQ, dK, dV,                                                          \
           {stride_qz, stride_qh, stride_qm, stride_qk}, {stride_kz, stride_kg, stride_kn, stride_kk},     \
           {stride_vz, stride_vg, stride_vn, stride_vk}, {stride_oz, stride_oh, stride_om, stride_ok},     \
           {stride_lz, stride_lh, stride_lm}, {stride_mz, stride_mh, stride_mm},                           \
           {stride_dqz, stride_dqh, stride_dqm, stride_dqk}, {stride_dkz, stride_dkg, stride_dkn, stride_dkk}, \
           {stride_dvz, stride_dvg, stride_dvn, stride_dvk}};

int nsa_sliding_window_fwd(const void* Q, const void* K, const void* V, void* Out, float sm_scale, float* L, float* M,
                           int64_t stride_qz, int64_t stride_qh, int64_t stride_qm, int64_t stride_qk,
                           int64_t stride_kz, int64_t stride_kg, int64_t stride_kn, int64_t stride_kk,
                           int64_t stride_vz, int64_t stride_vg, int64_t stride_vn, int64_t stride_vk,
                           int64_t stride_oz, int64_t stride_oh, int64_t stride_om, int64_t stride_ok,
                           int64_t stride_lz, int64_t stride_lh, int64_t stride_lm, int64_t stride_mz,
                           int64_t stride_mh, int64_t stride_mm, int Z, int H, int n_kv_groups, int n_ctx,
                           int window_size, int head_dim_qk, int head_dim_v, int dtype, void* workspace,
                           size_t workspace_bytes, nsa_stream_t stream) {
  NSA_FWD_IO
  Shape s{kSliding, dtype, Z, H, n_kv_groups, n_ctx, n_ctx, head_dim_qk, head_dim_v, 0, 64, window_size};
  return run_fwd(s, io, sm_scale, window_size, nullptr, nullptr, nullptr, 0, 0, 1, workspace, workspace_bytes,
                 (hipStream_t)stream);
}

int nsa_sliding_window_fwd_noalloc(const void* Q, const void* K, const void* V, void* Out, float sm_scale, float* L,
                                   float* M, int64_t stride_qz, int64_t stride_qh, int64_t stride_qm,
                                   int64_t stride_qk, int64_t stride_kz, int64_t stride_kg, int64_t stride_kn,
                                   int64_t stride_kk, int64_t stride_vz, int64_t stride_vg, int64_t stride_vn,
                                   int64_t stride_vk, int64_t stride_oz, int64_t stride_oh, int64_t stride_om,
                                   int64_t stride_ok, int64_t stride_lz, int64_t stride_lh, int64_t stride_lm,
                                   int64_t stride_mz, int64_t stride_mh, int64_t stride_mm, int Z, int H,
                                   int n_kv_groups, int n_ctx, int window_size, int head_dim_qk, int head_dim_v,
                                   int dtype, nsa_stream_t stream) {
  NSA_FWD_IO
  Shape s{kSliding, dtype, Z, H, n_kv_groups, n_ctx, n_ctx, head_dim_qk, head_dim_v, 0, 64, window_size};
  int rc = validate(s);
  if (rc) return rc;
  const size_t need = make_layout(s, false).total;
  if (need > kNoAllocScratchBytes)
    return fail(NSA_ERR_WORKSPACE,
                "nsa_sliding_window_fwd_noalloc: this shape needs %zu bytes of scratch, more than the %zu-byte "
                "static scratch; use nsa_sliding_window_fwd with a workspace",
                need, kNoAllocScratchBytes);
  void* ws = nullptr;
  if ((rc = scratch_ptr(&ws))) return rc;
  return run_fwd(s, io, sm_scale, window_size, nullptr, nullptr, nullptr, 0, 0, 1, ws, kNoAllocScratchBytes,
                 (hipStream_t)stream);
}

int nsa_sliding_window_bwd(const void* Q, const void* K, const void* V, const void* Out, const void* dOut,
                           float sm_scale, const float* L, const float* M, int64_t stride_qz, int64_t stride_qh,
                           int64_t stride_qm, int64_t stride_qk, int64_t stride_kz, int64_t stride_kg,
                           int64_t stride_kn, int64_t stride_kk, int64_t stride_vz, int64_t stride_vg,
                           int64_t stride_vn, int64_t stride_vk, int64_t stride_oz, int64_t stride_oh,
                           int64_t stride_om, int64_t stride_ok, int64_t stride_lz, int64_t stride_lh,
                           int64_t stride_lm, int64_t stride_mz, int64_t stride_mh, int64_t stride_mm, void* dQ,
                           void* dK, void* dV, int64_t stride_dqz, int64_t stride_dqh, int64_t stride_dqm,
                           int64_t stride_dqk, int64_t stride_dkz, int64_t stride_dkg, int64_t stride_dkn,
                           int64_t stride_dkk, int64_t stride_dvz, int64_t stride_dvg, int64_t stride_dvn,
                           int64_t stride_dvk, int Z, int H, int n_kv_groups, int n_ctx, int window_size,
                           int head_dim_qk, int head_dim_v, int dtype, void* workspace, size_t workspace_bytes,
                           nsa_stream_t stream) {
  NSA_BWD_IO
  Shape s{kSliding, dtype, Z, H, n_kv_groups, n_ctx, n_ctx, head_dim_qk, head_dim_v, 0, 64, window_size};
  return run_bwd(s, io, sm_scale, window_size, nullptr, nullptr, nullptr, 0, 0, 1, workspace, workspace_bytes,
                 (hipStream_t)stream);
}

int nsa_compression_fwd(const void* Q, const void* K, const void* V, const int32_t* Block_ends, void* Out,
                        float sm_scale, float* L, float* M, int64_t stride_qz, int64_t stride_qh, int64_t stride_qm,
                        int64_t stride_qk, int64_t stride_kz, int64_t stride_kg, int64_t stride_kn,
                        int64_t stride_kk, int64_t stride_vz, int64_t stride_vg, int64_t stride_vn,
                        int64_t stride_vk, int64_t stride_oz, int64_t stride_oh, int64_t stride_om,
                        int64_t stride_ok, int64_t stride_lz, int64_t stride_lh, int64_t stride_lm,
                        int64_t stride_mz, int64_t stride_mh, int64_t stride_mm, int Z, int H, int n_kv_groups,
                        int n_ctx_q, int n_blocks, int head_dim_qk, int head_dim_v, int dtype, void* workspace,
                        size_t workspace_bytes, nsa_stream_t stream) {
  NSA_FWD_IO
  Shape s{kCompression, dtype, Z, H, n_kv_groups, n_ctx_q, n_blocks, head_dim_qk, head_dim_v, 0, 64};
  if (n_blocks > 0 && !Block_ends) return fail(NSA_ERR_INVALID, "Block_ends is null");
  return run_fwd(s, io, sm_scale, 0, Block_ends, nullptr, nullptr, 0, 0, 1, workspace, workspace_bytes,
                 (hipStream_t)stream);
}

int nsa_compression_bwd(const void* Q, const void* K, const void* V, const int32_t* Block_ends, const void* Out,
                        const void* dOut, float sm_scale, const float* L, const float* M, int64_t stride_qz,
                        int64_t stride_qh, int64_t stride_qm, int64_t stride_qk, int64_t stride_kz,
                        int64_t stride_kg, int64_t stride_kn, int64_t stride_kk, int64_t stride_vz,
                        int64_t stride_vg, int64_t stride_vn, int64_t stride_vk, int64_t stride_oz,
                        int64_t stride_oh, int64_t stride_om, int64_t stride_ok, int64_t stride_lz,
                        int64_t stride_lh, int64_t stride_lm, int64_t stride_mz, int64_t stride_mh,
                        int64_t stride_mm, void* dQ, void* dK, void* dV, int64_t stride_dqz, int64_t stride_dqh,
                        int64_t stride_dqm, int64_t stride_dqk, int64_t stride_dkz, int64_t stride_dkg,
                        int64_t stride_dkn, int64_t stride_dkk, int64_t stride_dvz, int64_t stride_dvg,
                        int64_t stride_dvn, int64_t stride_dvk, int Z, int H, int n_kv_groups, int n_ctx_q,
                        int n_blocks, int head_dim_qk, int head_dim_v, int dtype, void* workspace,
                        size_t workspace_bytes, nsa_stream_t stream) {
  NSA_BWD_IO
  Shape s{kCompression, dtype, Z, H, n_kv_groups, n_ctx_q, n_blocks, head_dim_qk, head_dim_v, 0, 64};
  if (n_blocks > 0 && !Block_ends) return fail(NSA_ERR_INVALID, "Block_ends is null");
  return run_bwd(s, io, sm_scale, 0, Block_ends, nullptr, nullptr, 0, 0, 1, workspace, workspace_bytes,
                 (hipStream_t)stream);
}

int nsa_sparse_selection_fwd(const void* Q, const void* K, const void* V, const void* Block_indices, void* Out,
                             float sm_scale, float* L, float* M, int64_t stride_qz, int64_t stride_qh,
                             int64_t stride_qm, int64_t stride_qk, int64_t stride_kz, int64_t stride_kg,
                             int64_t stride_kn, int64_t stride_kk, int64_t stride_vz, int64_t stride_vg,
                             int64_t stride_vn, int64_t stride_vk, int64_t stride_oz, int64_t stride_oh,
                             int64_t stride_om, int64_t stride_ok, int64_t stride_bz, int64_t stride_bg,
                             int64_t stride_bm, int64_t stride_bn, int64_t stride_lz, int64_t stride_lh,
                             int64_t stride_lm, int64_t stride_mz, int64_t stride_mh, int64_t stride_mm, int Z, int H,
                             int n_kv_groups, int n_ctx_q, int n_ctx_kv, int n_slots, int block_size_selection,
                             int is_causal, int index_is_int64, int all_invalid_fallback, int head_dim_qk,
                             int head_dim_v, int dtype, void* workspace, size_t workspace_bytes,
                             nsa_stream_t stream) {
  NSA_FWD_IO
  Shape s{kSelection, dtype, Z, H, n_kv_groups, n_ctx_q, n_ctx_kv, head_dim_qk, head_dim_v, n_slots,
          block_size_selection};
  if (n_slots > 0 && n_ctx_q > 0 && !Block_indices) return fail(NSA_ERR_INVALID, "Block_indices is null");
  const int64_t sidx[4] = {stride_bz, stride_bg, stride_bm, stride_bn};
  return run_fwd(s, io, sm_scale, 0, nullptr, Block_indices, sidx, index_is_int64, all_invalid_fallback,
                 is_causal ? 1 : 0, workspace, workspace_bytes, (hipStream_t)stream);
}

int nsa_sparse_selection_bwd(const void* Q, const void* K, const void* V, const void* Block_indices, const void* Out,
                             const void* dOut, float sm_scale, const float* L, const float* M, int64_t stride_qz,
                             int64_t stride_qh, int64_t stride_qm, int64_t stride_qk, int64_t stride_kz,
                             int64_t stride_kg, int64_t stride_kn, int64_t stride_kk, int64_t stride_vz,
                             int64_t stride_vg, int64_t stride_vn, int64_t stride_vk, int64_t stride_oz,
                             int64_t stride_oh, int64_t stride_om, int64_t stride_ok, int64_t stride_bz,
                             int64_t stride_bg, int64_t stride_bm, int64_t stride_bn, int64_t stride_lz,
                             int64_t stride_lh, int64_t stride_lm, int64_t stride_mz, int64_t stride_mh,
                             int64_t stride_mm, void* dQ, void* dK, void* dV, int64_t stride_dqz, int64_t stride_dqh,
                             int64_t stride_dqm, int64_t stride_dqk, int64_t stride_dkz, int64_t stride_dkg,
                             int64_t stride_dkn, int64_t stride_dkk, int64_t stride_dvz, int64_t stride_dvg,
                             int64_t stride_dvn, int64_t stride_dvk, int Z, int H, int n_kv_groups, int n_ctx_q,
                             int n_ctx_kv, int n_slots, int block_size_selection, int is_causal, int index_is_int64,
                             int all_invalid_fallback, int head_dim_qk, int head_dim_v, int dtype, void* workspace,
                             size_t workspace_bytes, nsa_stream_t stream) {
  NSA_BWD_IO
  Shape s{kSelection, dtype, Z, H, n_kv_groups, n_ctx_q, n_ctx_kv, head_dim_qk, head_dim_v, n_slots,
          block_size_selection};
  if (n_slots > 0 && n_ctx_q > 0 && !Block_indices) return fail(NSA_ERR_INVALID, "Block_indices is null");
  const int64_t sidx[4] = {stride_bz, stride_bg, stride_bm, stride_bn};
  return run_bwd(s, io, sm_scale, 0, nullptr, Block_indices, sidx, index_is_int64, all_invalid_fallback,
                 is_causal ? 1 : 0, workspace, workspace_bytes, (hipStream_t)stream);
}

int nsa_sliding_window_bwd_ex(const void* Q, const void* K, const void* V, const void* Out, const void* dOut,
                           float sm_scale, const float* L, const float* M, int64_t stride_qz, int64_t stride_qh,
                           int64_t stride_qm, int64_t stride_qk, int64_t stride_kz, int64_t stride_kg,
                           int64_t stride_kn, int64_t stride_kk, int64_t stride_vz, int64_t stride_vg,
                           int64_t stride_vn, int64_t stride_vk, int64_t stride_oz, int64_t stride_oh,
                           int64_t stride_om, int64_t stride_ok, int64_t stride_lz, int64_t stride_lh,
                           int64_t stride_lm, int64_t stride_mz, int64_t stride_mh, int64_t stride_mm, void* dQ,
                           void* dK, void* dV, int64_t stride_dqz, int64_t stride_dqh, int64_t stride_dqm,
                           int64_t stride_dqk, int64_t stride_dkz, int64_t stride_dkg, int64_t stride_dkn,
                           int64_t stride_dkk, int64_t stride_dvz, int64_t stride_dvg, int64_t stride_dvn,
                           int64_t stride_dvk, int Z, int H, int n_kv_groups, int n_ctx, int window_size,
                           int head_dim_qk, int head_dim_v, int dtype,
                           int bwd_flags, const float* delta_in, const float* row_gate, float* row_dot, void* workspace, size_t workspace_bytes,
                           nsa_stream_t stream) {
  NSA_BWD_IO
  if (int rc = set_bwd_ext(io, bwd_flags, delta_in, row_gate, row_dot)) return rc;
  Shape s{kSliding, dtype, Z, H, n_kv_groups, n_ctx, n_ctx, head_dim_qk, head_dim_v, 0, 64, window_size};
  return run_bwd(s, io, sm_scale, window_size, nullptr, nullptr, nullptr, 0, 0, 1, workspace, workspace_bytes,
                 (hipStream_t)stream);
}

int nsa_sliding_window_bwd_pair(const void* Q, const void* K, const void* V, const void* Out, const void* dOut,
                                float sm_scale, const float* L, const float* M, int64_t stride_qz,
                                int64_t stride_qh, int64_t stride_qm, int64_t stride_qk, int64_t stride_kz,
                                int64_t stride_kg, int64_t stride_kn, int64_t stride_kk, int64_t stride_vz,
                                int64_t stride_vg, int64_t stride_vn, int64_t stride_vk, int64_t stride_oz,
                                int64_t stride_oh, int64_t stride_om, int64_t stride_ok, int64_t stride_lz,
                                int64_t stride_lh, int64_t stride_lm, int64_t stride_mz, int64_t stride_mh,
                                int64_t stride_mm, void* dQ, void* dK, void* dV, int64_t stride_dqz,
                                int64_t stride_dqh, int64_t stride_dqm, int64_t stride_dqk, int64_t stride_dkz,
                                int64_t stride_dkg, int64_t stride_dkn, int64_t stride_dkk, int64_t stride_dvz,
                                int64_t stride_dvg, int64_t stride_dvn, int64_t stride_dvk, int Z, int H,
                                int n_kv_groups, int n_ctx, int window_size, int head_dim_qk, int head_dim_v,
                                int dtype, int bwd_flags, const float* delta_in, const float* row_gate,
                                float* row_dot, const int32_t* cmp_block_ends, int cmp_n_blocks,
                                const void* cmp_workspace, size_t cmp_workspace_bytes, void* workspace,
                                size_t workspace_bytes, nsa_stream_t stream) {
  NSA_BWD_IO
  if (int rc = set_bwd_ext(io, bwd_flags, delta_in, row_gate, row_dot)) return rc;
  if (io.defer_dq) return fail(NSA_ERR_INVALID, "the paired backward runs its dQ kernel (no NSA_BWD_DQ_DEFER)");
  if (!cmp_workspace) return fail(NSA_ERR_INVALID, "cmp_workspace is null");
  io.pair_ws = cmp_workspace;
  io.pair_ws_bytes = cmp_workspace_bytes;
  io.pair_block_ends = cmp_block_ends;
  io.pair_n_blocks = cmp_n_blocks;
  Shape s{kSliding, dtype, Z, H, n_kv_groups, n_ctx, n_ctx, head_dim_qk, head_dim_v, 0, 64, window_size};
  return run_bwd(s, io, sm_scale, window_size, nullptr, nullptr, nullptr, 0, 0, 1, workspace, workspace_bytes,
                 (hipStream_t)stream);
}

int nsa_compression_bwd_ex(const void* Q, const void* K, const void* V, const int32_t* Block_ends, const void* Out,
                        const void* dOut, float sm_scale, const float* L, const float* M, int64_t stride_qz,
                        int64_t stride_qh, int64_t stride_qm, int64_t stride_qk, int64_t stride_kz,
                        int64_t stride_kg, int64_t stride_kn, int64_t stride_kk, int64_t stride_vz,
                        int64_t stride_vg, int64_t stride_vn, int64_t stride_vk, int64_t stride_oz,
                        int64_t stride_oh, int64_t stride_om, int64_t stride_ok, int64_t stride_lz,
                        int64_t stride_lh, int64_t stride_lm, int64_t stride_mz, int64_t stride_mh,
                        int64_t stride_mm, void* dQ, void* dK, void* dV, int64_t stride_dqz, int64_t stride_dqh,
                        int64_t stride_dqm, int64_t stride_dqk, int64_t stride_dkz, int64_t stride_dkg,
                        int64_t stride_dkn, int64_t stride_dkk, int64_t stride_dvz, int64_t stride_dvg,
                        int64_t stride_dvn, int64_t stride_dvk, int Z, int H, int n_kv_groups, int n_ctx_q,
                        int n_blocks, int head_dim_qk, int head_dim_v, int dtype,
                        int bwd_flags, const float* delta_in, const float* row_gate, float* row_dot, void* workspace,
                        size_t workspace_bytes, nsa_stream_t stream) {
  NSA_BWD_IO
  if (int rc = set_bwd_ext(io, bwd_flags, delta_in, row_gate, row_dot)) return rc;
  Shape s{kCompression, dtype, Z, H, n_kv_groups, n_ctx_q, n_blocks, head_dim_qk, head_dim_v, 0, 64};
  if (n_blocks > 0 && !Block_ends) return fail(NSA_ERR_INVALID, "Block_ends is null");
  return run_bwd(s, io, sm_scale, 0, Block_ends, nullptr, nullptr, 0, 0, 1, workspace, workspace_bytes,
                 (hipStream_t)stream);
}

int nsa_sparse_selection_bwd_ex(const void* Q, const void* K, const void* V, const void* Block_indices, const void* Out,
                             const void* dOut, float sm_scale, const float* L, const float* M, int64_t stride_qz,
                             int64_t stride_qh, int64_t stride_qm, int64_t stride_qk, int64_t stride_kz,
                             int64_t stride_kg, int64_t stride_kn, int64_t stride_kk, int64_t stride_vz,
                             int64_t stride_vg, int64_t stride_vn, int64_t stride_vk, int64_t stride_oz,
                             int64_t stride_oh, int64_t stride_om, int64_t stride_ok, int64_t stride_bz,
                             int64_t stride_bg, int64_t stride_bm, int64_t stride_bn, int64_t stride_lz,
                             int64_t stride_lh, int64_t stride_lm, int64_t stride_mz, int64_t stride_mh,
                             int64_t stride_mm, void* dQ, void* dK, void* dV, int64_t stride_dqz, int64_t stride_dqh,
                             int64_t stride_dqm, int64_t stride_dqk, int64_t stride_dkz, int64_t stride_dkg,
                             int64_t stride_dkn, int64_t stride_dkk, int64_t stride_dvz, int64_t stride_dvg,
                             int64_t stride_dvn, int64_t stride_dvk, int Z, int H, int n_kv_groups, int n_ctx_q,
                             int n_ctx_kv, int n_slots, int block_size_selection, int is_causal, int index_is_int64,
                             int all_invalid_fallback, int head_dim_qk, int head_dim_v, int dtype,
                             int bwd_flags, const float* delta_in, const float* row_gate, float* row_dot, void* workspace,
                             size_t workspace_bytes, nsa_stream_t stream) {
  NSA_BWD_IO
  if (int rc = set_bwd_ext(io, bwd_flags, delta_in, row_gate, row_dot)) return rc;
  Shape s{kSelection, dtype, Z, H, n_kv_groups, n_ctx_q, n_ctx_kv, head_dim_qk, head_dim_v, n_slots,
          block_size_selection};
  if (n_slots > 0 && n_ctx_q > 0 && !Block_indices) return fail(NSA_ERR_INVALID, "Block_indices is null");
  const int64_t sidx[4] = {stride_bz, stride_bg, stride_bm, stride_bn};
  return run_bwd(s, io, sm_scale, 0, nullptr, Block_indices, sidx, index_is_int64, all_invalid_fallback,
                 is_causal ? 1 : 0, workspace, workspace_bytes, (hipStream_t)stream);
}

int nsa_sliding_window_fwd_ex(const void* Q, const void* K, const void* V, void* Out, float sm_scale, float* L,
float* M,
                           int64_t stride_qz, int64_t stride_qh, int64_t stride_qm, int64_t stride_qk,
                           int64_t stride_kz, int64_t stride_kg, int64_t stride_kn, int64_t stride_kk,
                           int64_t stride_vz, int64_t stride_vg, int64_t stride_vn, int64_t stride_vk,
                           int64_t stride_oz, int64_t stride_oh, int64_t stride_om, int64_t stride_ok,
                           int64_t stride_lz, int64_t stride_lh, int64_t stride_lm, int64_t stride_mz,
                           int64_t stride_mh, int64_t stride_mm, int Z, int H, int n_kv_groups, int n_ctx,
                           int window_size, int head_dim_qk, int head_dim_v, int dtype, int n_ctx_kv, int q_offset,
                           const void* mix_o0, const void* mix_o1, const float* mix_gates, void* mix_out,
                           int64_t stride_xz, int64_t stride_xh, int64_t stride_xm, void* workspace,
                           size_t workspace_bytes, nsa_stream_t stream) {
  NSA_FWD_IO
  io.mix_o0 = mix_o0;
  io.mix_o1 = mix_o1;
  io.mix_gates = mix_gates;
  io.mix_out = mix_out;
  io.sx[0] = stride_xz;
  io.sx[1] = stride_xh;
  io.sx[2] = stride_xm;
  Shape s{kSliding, dtype, Z, H, n_kv_groups, n_ctx, n_ctx_kv, head_dim_qk, head_dim_v, 0, 64, window_size};
  s.q0 = q_offset;
  return run_fwd(s, io, sm_scale, window_size, nullptr, nullptr, nullptr, 0, 0, 1, workspace, workspace_bytes,
                 (hipStream_t)stream);
}

int nsa_compression_fwd_ex(const void* Q, const void* K, const void* V, const int32_t* Block_ends, void* Out,
                        float sm_scale, float* L, float* M, int64_t stride_qz, int64_t stride_qh, int64_t stride_qm,
                        int64_t stride_qk, int64_t stride_kz, int64_t stride_kg, int64_t stride_kn,
                        int64_t stride_kk, int64_t stride_vz, int64_t stride_vg, int64_t stride_vn,
                        int64_t stride_vk, int64_t stride_oz, int64_t stride_oh, int64_t stride_om,
                        int64_t stride_ok, int64_t stride_lz, int64_t stride_lh, int64_t stride_lm,
                        int64_t stride_mz, int64_t stride_mh, int64_t stride_mm, int Z, int H, int n_kv_groups,
                        int n_ctx_q, int n_blocks, int head_dim_qk, int head_dim_v, int dtype, int q_offset,
                        void* workspace,
                        size_t workspace_bytes, nsa_stream_t stream) {
  NSA_FWD_IO
  Shape s{kCompression, dtype, Z, H, n_kv_groups, n_ctx_q, n_blocks, head_dim_qk, head_dim_v, 0, 64};
  s.q0 = q_offset;
  if (n_blocks > 0 && !Block_ends) return fail(NSA_ERR_INVALID, "Block_ends is null");
  return run_fwd(s, io, sm_scale, 0, Block_ends, nullptr, nullptr, 0, 0, 1, workspace, workspace_bytes,
                 (hipStream_t)stream);
}

int nsa_sparse_selection_fwd_ex(const void* Q, const void* K, const void* V, const void* Block_indices, void* Out,
                             float sm_scale, float* L, float* M, int64_t stride_qz, int64_t stride_qh,
                             int64_t stride_qm, int64_t stride_qk, int64_t stride_kz, int64_t stride_kg,
                             int64_t stride_kn, int64_t stride_kk, int64_t stride_vz, int64_t stride_vg,
                             int64_t stride_vn, int64_t stride_vk, int64_t stride_oz, int64_t stride_oh,
                             int64_t stride_om, int64_t stride_ok, int64_t stride_bz, int64_t stride_bg,
                             int64_t stride_bm, int64_t stride_bn, int64_t stride_lz, int64_t stride_lh,
                             int64_t stride_lm, int64_t stride_mz, int64_t stride_mh, int64_t stride_mm, int Z, int H,
                             int n_kv_groups, int n_ctx_q, int n_ctx_kv, int n_slots, int block_size_selection,
                             int is_causal, int index_is_int64, int all_invalid_fallback, int head_dim_qk,
                             int head_dim_v, int dtype, int q_offset, void* workspace, size_t workspace_bytes,
                             nsa_stream_t stream) {
  NSA_FWD_IO
  Shape s{kSelection, dtype, Z, H, n_kv_groups, n_ctx_q, n_ctx_kv, head_dim_qk, head_dim_v, n_slots,
          block_size_selection};
  s.q0 = q_offset;
  if (n_slots > 0 && n_ctx_q > 0 && !Block_indices) return fail(NSA_ERR_INVALID, "Block_indices is null");
  const int64_t sidx[4] = {stride_bz, stride_bg, stride_bm, stride_bn};
  return run_fwd(s, io, sm_scale, 0, nullptr, Block_indices, sidx, index_is_int64, all_invalid_fallback,
                 is_causal ? 1 : 0, workspace, workspace_bytes, (hipStream_t)stream);
}

}  // extern "C"
