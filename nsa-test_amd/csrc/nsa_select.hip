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
constexpr int kCsrChunk = 256;  // timesteps per fill chunk

__global__ void zero_ints_kernel(int* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

__global__ __launch_bounds__(256) void sel_clean_kernel(const void* idx, int idx_is64, int64_t si_b, int64_t si_g,
                                                        int64_t si_t, int64_t si_n, int G, int Tq, int n_in,
                                                        int nslots, int lprime, int nblk, int fallback, int causal,
                                                        int* clean, int* chunk_cnt, int nchunks) {
  const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t nrows = (int64_t)gridDim.y * Tq;  // gridDim.y = B*G
  const int bg = blockIdx.y;
  if (row >= Tq) return;
  (void)nrows;
  const int t = (int)row;
  const int b = bg / G, g = bg % G;
  int vals[kCleanMaxSlots];
  int n = 0;
  bool any_valid = false;
  for (int s = 0; s < n_in; ++s) {
    const int64_t off = b * si_b + g * si_g + (int64_t)t * si_t + s * si_n;
    const int64_t v = idx_is64 ? reinterpret_cast<const int64_t*>(idx)[off] : reinterpret_cast<const int*>(idx)[off];
    if (v >= 0) any_valid = true;
    vals[s] = (int)(v < -1 ? -1 : (v > 0x3fffffff ? 0x3fffffff : v));
  }
  if (fallback && !any_valid && n_in > 0) {
    for (int s = 0; s < n_in; ++s) vals[s] = t / lprime;
  }
  // filter + insertion sort with de-duplication
  int out[kCleanMaxSlots];
  for (int s = 0; s < n_in; ++s) {
    const int v = vals[s];
    if (v < 0 || v >= nblk) continue;
    if (causal && (int64_t)v * lprime > t) continue;
    int p = n;
    bool dup = false;
    while (p > 0 && out[p - 1] >= v) {
      if (out[p - 1] == v) {
        dup = true;
        break;
      }
      --p;
    }
    if (dup) continue;
    for (int q = n; q > p; --q) out[q] = out[q - 1];
    out[p] = v;
    ++n;
  }
  int* dst = clean + ((int64_t)bg * Tq + t) * nslots;
  for (int s = 0; s < nslots; ++s) dst[s] = s < n ? out[s] : -1;
  if (chunk_cnt) {
    int* cc = chunk_cnt + ((int64_t)bg * nchunks + t / kCsrChunk) * nblk;
    for (int s = 0; s < n; ++s) atomicAdd(&cc[out[s]], 1);
  }
}

// Per (b,g): chunk_cnt[c][j] -> exclusive running base over chunks (+ block offset);
// csr_off[j] = exclusive scan of block totals; seg_off[j] = exclusive scan of
// ceil(total_j / kSegT) work items.
__global__ __launch_bounds__(256) void sel_csr_scan_kernel(int* chunk_cnt, int nchunks, int nblk, int* csr_off,
                                                           int* seg_off) {
  extern __shared__ int tot[];  // nblk
  const int bg = blockIdx.x;
  int* cc = chunk_cnt + (int64_t)bg * nchunks * nblk;
  for (int j = threadIdx.x; j < nblk; j += 256) {
    int run = 0;
    for (int c = 0; c < nchunks; ++c) {
      const int x = cc[(int64_t)c * nblk + j];
      cc[(int64_t)c * nblk + j] = run;
      run += x;
    }
    tot[j] = run;
  }
  __syncthreads();
  int* off = csr_off + (int64_t)bg * (nblk + 1);
  int* so = seg_off + (int64_t)bg * (nblk + 1);
  if (threadIdx.x == 0) {
    int run = 0, srun = 0;
    for (int j = 0; j < nblk; ++j) {
      off[j] = run;
      so[j] = srun;
      run += tot[j];
      srun += (tot[j] + kSegT - 1) / kSegT;
      tot[j] = off[j];
    }
    off[nblk] = run;
    so[nblk] = srun;
  }
  __syncthreads();
  for (int j = threadIdx.x; j < nblk; j += 256) {
    const int base = tot[j];
    for (int c = 0; c < nchunks; ++c) cc[(int64_t)c * nblk + j] += base;
  }
}

// One wave per (b, g, chunk of kCsrChunk timesteps): walk the timesteps in order,
// appending t to each of its blocks' lists.  A block appears at most once per row,
// so the lanes of one step never collide.
__global__ __launch_bounds__(64) void sel_csr_fill_kernel(const int* clean, const int* chunk_base, int Tq,
                                                          int nslots, int nchunks, int nblk, int* csr_t,
                                                          int64_t csr_stride) {
  extern __shared__ int cur[];  // nblk
  const int c = blockIdx.x, bg = blockIdx.y;
  const int lane = threadIdx.x;
  const int* cb = chunk_base + ((int64_t)bg * nchunks + c) * nblk;
  for (int j = lane; j < nblk; j += 64) cur[j] = cb[j];
  __syncthreads();
  int* out = csr_t + (int64_t)bg * csr_stride;
  const int t0 = c * kCsrChunk;
  const int t1 = min(Tq, t0 + kCsrChunk);
  for (int t = t0; t < t1; ++t) {
    const int* row = clean + ((int64_t)bg * Tq + t) * nslots;
    for (int s = lane; s < nslots; s += 64) {
      const int v = row[s];
      if (v >= 0) {
        const int pos = cur[v];
        out[pos] = t;
        cur[v] = pos + 1;
      }
    }
    __syncthreads();
  }
}

void launch_sel_clean(const void* idx, int idx_is64, int64_t si_b, int64_t si_g, int64_t si_t, int64_t si_n, int B,
                      int G, int Tq, int n_in, int nslots, int lprime, int Tkv, int fallback, int causal, int* clean,
                      int* chunk_cnt, int nblk, hipStream_t st) {
  const int nchunks = (Tq + kCsrChunk - 1) / kCsrChunk;
  if (chunk_cnt) {
    const int64_t n = (int64_t)B * G * nchunks * nblk;
    hipLaunchKernelGGL(zero_ints_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, chunk_cnt, n);
  }
  (void)Tkv;
  dim3 grid((Tq + 255) / 256, B * G);
  hipLaunchKernelGGL(sel_clean_kernel, grid, dim3(256), 0, st, idx, idx_is64, si_b, si_g, si_t, si_n, G, Tq, n_in,
                     nslots, lprime, nblk, fallback, causal, clean, chunk_cnt, nchunks);
}

void launch_sel_csr(const int* clean, int* chunk_cnt, int B, int G, int Tq, int nslots, int nblk, int* csr_off,
                    int* csr_t, int* seg_off, hipStream_t st) {
  const int nchunks = (Tq + kCsrChunk - 1) / kCsrChunk;
  hipLaunchKernelGGL(sel_csr_scan_kernel, dim3(B * G), dim3(256), nblk * sizeof(int), st, chunk_cnt, nchunks, nblk,
                     csr_off, seg_off);
  hipLaunchKernelGGL(sel_csr_fill_kernel, dim3(nchunks, B * G), dim3(64), nblk * sizeof(int), st, clean, chunk_cnt,
                     Tq, nslots, nchunks, nblk, csr_t, (int64_t)Tq * nslots);
}

int sel_csr_chunks(int Tq) { return (Tq + kCsrChunk - 1) / kCsrChunk; }

}  // namespace nsa
