// Host-side launchers behind the C ABI (internal, not exported).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "nsa_attn.h"

// Head-dimension pairs (DK, DV) with compiled kernels.  Other widths are served by
// zero-padding to the next pair in the host shim (padding q/k columns with zeros
// leaves q.k unchanged; padded v columns are dropped).
#define NSA_HEAD_DIMS(X) X(32, 32) X(64, 64) X(128, 128) X(192, 128)

namespace nsa {

void launch_repack(int dtype, const void* src, int64_t s_b, int64_t s_g, int64_t s_r, int64_t s_c, int B, int G,
                   int R, int C, int Rp, void* rowm, void* colm, void* rowf, void* colf, hipStream_t st);
// K and V fragment copies of one call (one launch when both suit the fragment kernel);
// sk / sv: (b, g, row, feature) strides
void launch_repack_kv(int dtype, const void* k, const int64_t* sk, int dk, void* krf, void* kcf, const void* v,
                      const int64_t* sv, int dv, void* vrf, void* vcf, int B, int G, int R, int Rp, hipStream_t st);

// return false when (dtype, dk, dv, branch) has no compiled kernel
bool dispatch_attn_fwd(int dtype, int dk, int dv, int br, const AttnArgs& a, hipStream_t st);
bool dispatch_attn_bwd_dq(int dtype, int dk, int dv, int br, const AttnArgs& a, hipStream_t st);
bool dispatch_attn_bwd_dkdv(int dtype, int dk, int dv, int br, const AttnArgs& a, hipStream_t st);
// lse2 / delta (/ row_dot) of every query row before a dK/dV kernel that runs first
bool launch_row_stats(int dtype, int dv, const AttnArgs& a, hipStream_t st);
void launch_partial_reduce(int dtype, int dk, int dv, int br, const AttnArgs& a, hipStream_t st);
// dK / dV [B, G, Tkv, dk | dv] (a.dk / a.dv, any strides) set to zero
void launch_zero_dkdv(int dtype, int dk, int dv, const AttnArgs& a, hipStream_t st);

// selection index cleaning and block -> query CSR
void launch_sel_clean(const void* idx, int idx_is64, int64_t si_b, int64_t si_g, int64_t si_t, int64_t si_n, int B,
                      int G, int Tq, int n_in, int nslots, int lprime, int Tkv, int fallback, int causal, int* clean,
                      int* chunk_cnt, int nblk, int q0, hipStream_t st);
// csr_s (nullable) receives each entry's slot in its timestep's cleaned list
void launch_sel_csr(const int* clean, int* chunk_cnt, int B, int G, int Tq, int nslots, int nblk, int* csr_off,
                    int* csr_t, int* csr_s, int* seg_off, int seg, hipStream_t st);
int sel_csr_chunks(int Tq);

// record an error message for nsa_last_error(); returns `code`
int set_error(int code, const char* msg);

// Kernel ids for nsa_timing_begin (fwd / dq / dkdv are offset by the branch).
enum KernelId : int {
  kIdFwd = 0,    // + branch
  kIdDq = 3,     // + branch
  kIdDkdv = 6,   // + branch
  kIdReduce = 9,
  kIdScore = 10,
  kIdPoolFwd = 11,
  kIdPoolBwd = 12,
  kIdPrep = 13,  // K/V repack, row statistics, selection index CSR
};

// Records a HIP event pair around its lifetime when timing of `kind` is armed.
class TimingScope {
 public:
  TimingScope(int kind, hipStream_t st);
  ~TimingScope();

 private:
  bool active_;
  hipStream_t stream_;
};

}  // namespace nsa
