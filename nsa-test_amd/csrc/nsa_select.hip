// Selection bookkeeping on the GPU.
//
// sel_clean: per (b, g, t) row, turn the caller's top-n slots into the set the
//   attention kernels iterate: drop -1 padding, blocks past the sequence and (when
//   causal) blocks that start after t; remove repeats (the reference oracle takes the
//   union of the selected blocks, nsa/reference.py:233-246); sort ascending.  With
//   `fallback` set, a row whose slots are all negative selects the block holding t,
//   as the autograd wrapper does (nsa/kernels.py:199-205).
// sel_csr:  invert the row -> blocks map into block -> ascending query timesteps
//   (a CSR per (b, g)), so the dK/dV kernels can own a key block each and reduce
//   over its queries in a fixed order: deterministic, no floating-point atomics.
#include "nsa_attn.h"
#include "nsa_kernels.h"

namespace nsa {

constexpr int kCleanMaxSlots = 64;
constexpr int kCsrChunk = 64;  // timesteps per fill chunk

__global__ void zero_ints_kernel(int* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

// SEG lanes (a power of two >= the slot count) clean one row: lane s holds slot s.  The
// kept value of a lane is its slot unless it is invalid or repeats an earlier slot;
// its position in the ascending output is the number of kept values below it.
template <int SEG>
__global__ __launch_bounds__(256) void sel_clean_kernel(const void* idx, int idx_is64, int64_t si_b, int64_t si_g,
                                                        int64_t si_t, int64_t si_n, int G, int Tq, int n_in,
                                                        int nslots, int lprime, int nblk, int fallback, int causal,
                                                        int* clean, int* chunk_cnt, int nchunks, int q0) {
  constexpr int kNone = 0x7fffffff;
  const int t = (int)(((int64_t)blockIdx.x * 256 + threadIdx.x) / SEG);
  const int s = threadIdx.x % SEG;
  const int bg = blockIdx.y;
  const int b = bg / G, g = bg % G;
  const bool row_ok = t < Tq;  // lanes past the last row take part in the shuffles only
  int raw = -1;
  if (row_ok && s < n_in) {
    const int64_t off = b * si_b + g * si_g + (int64_t)t * si_t + s * si_n;
    const int64_t v = idx_is64 ? reinterpret_cast<const int64_t*>(idx)[off] : reinterpret_cast<const int*>(idx)[off];
    raw = (int)(v < -1 ? -1 : (v > 0x3fffffff ? 0x3fffffff : v));
  }
  int any_valid = raw >= 0;
#pragma unroll
  for (int o = 1; o < SEG; o <<= 1) any_valid |= __shfl_xor(any_valid, o, SEG);
  const int ta = t + q0;  // absolute position of row t
  if (fallback && !any_valid && s < n_in) raw = ta / lprime;
  const bool ok = row_ok && raw >= 0 && raw < nblk && !(causal && (int64_t)raw * lprime > ta);
  const int key = ok ? raw : kNone;
  bool dup = false;
#pragma unroll
  for (int j = 0; j < SEG; ++j) {
    const int o = __shfl(key, j, SEG);
    dup |= j < s && o == key;
  }
  const bool keep = key != kNone && !dup;
  int pos = 0, nkept = 0;
#pragma unroll
  for (int j = 0; j < SEG; ++j) {
    const int o = __shfl(keep ? key : kNone, j, SEG);
    pos += o < key;
    nkept += o != kNone;
  }
  if (!row_ok) return;
  int* dst = clean + ((int64_t)bg * Tq + t) * nslots;
  if (keep) dst[pos] = key;
  for (int q = nkept + s; q < nslots; q += SEG) dst[q] = -1;
  if (chunk_cnt && keep) atomicAdd(&chunk_cnt[((int64_t)bg * nchunks + t / kCsrChunk) * nblk + key], 1);
}

// One wave per (b, g, block j): chunk_cnt[c][j] -> the exclusive running count of
// block j's entries in the chunks before c (64 chunks per step, a wave prefix sum);
// block j's total goes to tot[j].
__global__ __launch_bounds__(256) void sel_csr_chunk_scan_kernel(int* chunk_cnt, int nchunks, int nblk, int* tot) {
  const int lane = threadIdx.x & 63;
  const int j = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int bg = blockIdx.y;
  if (j >= nblk) return;  // whole wave
  int* cc = chunk_cnt + (int64_t)bg * nchunks * nblk + j;
  int carry = 0;
  for (int c0 = 0; c0 < nchunks; c0 += 64) {
    const int c = c0 + lane;
    const int x = c < nchunks ? cc[(int64_t)c * nblk] : 0;
    int inc = x;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(inc, o);
      if (lane >= o) inc += y;
    }
    if (c < nchunks) cc[(int64_t)c * nblk] = carry + inc - x;
    carry += __shfl(inc, 63);
  }
  if (lane == 0) tot[(int64_t)bg * (nblk + 1) + j] = carry;
}

// One workgroup per (b, g): csr_off[j] = exclusive prefix of the block totals (read
// from csr_off itself, where the chunk scan left them), seg_off[j] = exclusive prefix
// of ceil(total_j / seg) work items; entry nblk holds the sums.
__global__ __launch_bounds__(256) void sel_csr_block_scan_kernel(int nblk, int seg, int* csr_off, int* seg_off) {
  __shared__ int s_a[256], s_b[256];
  const int tid = threadIdx.x;
  const int bg = blockIdx.x;
  int* off = csr_off + (int64_t)bg * (nblk + 1);
  int* so = seg_off + (int64_t)bg * (nblk + 1);
  const int per = (nblk + 255) / 256;  // contiguous entries per thread
  const int j0 = min(nblk, tid * per), j1 = min(nblk, j0 + per);
  int sa = 0, sb = 0;
  for (int j = j0; j < j1; ++j) {
    const int t = off[j];
    sa += t;
    sb += (t + seg - 1) / seg;
  }
  s_a[tid] = sa;
  s_b[tid] = sb;
  __syncthreads();
  for (int o = 1; o < 256; o <<= 1) {  // inclusive scan over the 256 partials
    const int xa = tid >= o ? s_a[tid - o] : 0, xb = tid >= o ? s_b[tid - o] : 0;
    __syncthreads();
    s_a[tid] += xa;
    s_b[tid] += xb;
    __syncthreads();
  }
  int ra = s_a[tid] - sa, rb = s_b[tid] - sb;  // exclusive bases of this thread's range
  for (int j = j0; j < j1; ++j) {
    const int t = off[j];
    off[j] = ra;
    so[j] = rb;
    ra += t;
    rb += (t + seg - 1) / seg;
  }
  if (tid == 255) {
    off[nblk] = s_a[255];
    so[nblk] = s_b[255];
  }
}

// One wave per (b, g, chunk of kCsrChunk timesteps): walk the timesteps in order,
// appending t to each of its blocks' lists.  A block appears at most once per row,
// so the lanes of one step never collide.
__global__ __launch_bounds__(64) void sel_csr_fill_kernel(const int* clean, const int* chunk_base,
                                                          const int* csr_off, int Tq, int nslots, int nchunks,
                                                          int nblk, int* csr_t, int* csr_s, int64_t csr_stride) {
  extern __shared__ int cur[];  // nblk
  const int c = blockIdx.x, bg = blockIdx.y;
  const int lane = threadIdx.x;
  const int* cb = chunk_base + ((int64_t)bg * nchunks + c) * nblk;
  const int* off = csr_off + (int64_t)bg * (nblk + 1);
  for (int j = lane; j < nblk; j += 64) cur[j] = off[j] + cb[j];
  __syncthreads();
  int* out = csr_t + (int64_t)bg * csr_stride;
  int* out_s = csr_s ? csr_s + (int64_t)bg * csr_stride : nullptr;
  const int t0 = c * kCsrChunk;
  const int t1 = min(Tq, t0 + kCsrChunk);
  for (int t = t0; t < t1; ++t) {
    const int* row = clean + ((int64_t)bg * Tq + t) * nslots;
    for (int s = lane; s < nslots; s += 64) {
      const int v = row[s];
      if (v >= 0) {
        const int pos = cur[v];
        out[pos] = t;
        if (out_s) out_s[pos] = s;
        cur[v] = pos + 1;
      }
    }
    __syncthreads();
  }
}

void launch_sel_clean(const void* idx, int idx_is64, int64_t si_b, int64_t si_g, int64_t si_t, int64_t si_n, int B,
                      int G, int Tq, int n_in, int nslots, int lprime, int Tkv, int fallback, int causal, int* clean,
                      int* chunk_cnt, int nblk, int q0, hipStream_t st) {
  const int nchunks = (Tq + kCsrChunk - 1) / kCsrChunk;
  if (chunk_cnt) {
    const int64_t n = (int64_t)B * G * nchunks * nblk;
    hipLaunchKernelGGL(zero_ints_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, chunk_cnt, n);
  }
  (void)Tkv;
  // lanes per row: the smallest power of two >= the slot count (at most kCleanMaxSlots)
  const int seg = n_in <= 16 ? 16 : n_in <= 32 ? 32 : 64;
  dim3 grid((unsigned)(((int64_t)Tq * seg + 255) / 256), B * G);
  if (seg == 16)
    hipLaunchKernelGGL(sel_clean_kernel<16>, grid, dim3(256), 0, st, idx, idx_is64, si_b, si_g, si_t, si_n, G, Tq,
                       n_in, nslots, lprime, nblk, fallback, causal, clean, chunk_cnt, nchunks, q0);
  else if (seg == 32)
    hipLaunchKernelGGL(sel_clean_kernel<32>, grid, dim3(256), 0, st, idx, idx_is64, si_b, si_g, si_t, si_n, G, Tq,
                       n_in, nslots, lprime, nblk, fallback, causal, clean, chunk_cnt, nchunks, q0);
  else
    hipLaunchKernelGGL(sel_clean_kernel<64>, grid, dim3(256), 0, st, idx, idx_is64, si_b, si_g, si_t, si_n, G, Tq,
                       n_in, nslots, lprime, nblk, fallback, causal, clean, chunk_cnt, nchunks, q0);
}

void launch_sel_csr(const int* clean, int* chunk_cnt, int B, int G, int Tq, int nslots, int nblk, int* csr_off,
                    int* csr_t, int* csr_s, int* seg_off, int seg, hipStream_t st) {
  const int nchunks = (Tq + kCsrChunk - 1) / kCsrChunk;
  hipLaunchKernelGGL(sel_csr_chunk_scan_kernel, dim3((nblk + 3) / 4, B * G), dim3(256), 0, st, chunk_cnt, nchunks,
                     nblk, csr_off);
  hipLaunchKernelGGL(sel_csr_block_scan_kernel, dim3(B * G), dim3(256), 0, st, nblk, seg, csr_off, seg_off);
  hipLaunchKernelGGL(sel_csr_fill_kernel, dim3(nchunks, B * G), dim3(64), nblk * sizeof(int), st, clean, chunk_cnt,
                     csr_off, Tq, nslots, nchunks, nblk, csr_t, csr_s, (int64_t)Tq * nslots);
}

int sel_csr_chunks(int Tq) { return (Tq + kCsrChunk - 1) / kCsrChunk; }

}  // namespace nsa
