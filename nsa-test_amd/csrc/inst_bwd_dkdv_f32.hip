// Instantiations: attention bwd_dkdv kernels, element type float, every (DK, DV, branch).
#include "nsa_attn_bwd_dkdv.h"
#include "nsa_kernels.h"

namespace nsa {

bool dispatch_attn_bwd_dkdv_f32(int dk, int dv, int br, const AttnArgs& a, hipStream_t st) {
#define NSA_CASE(DKV, DVV)                                                          \
  if (dk == DKV && dv == DVV) {                                                    \
    if (br == kSliding) launch_attn_bwd_dkdv<float, DKV, DVV, kSliding>(a, st);         \
    else if (br == kCompression) launch_attn_bwd_dkdv<float, DKV, DVV, kCompression>(a, st); \
    else launch_attn_bwd_dkdv<float, DKV, DVV, kSelection>(a, st);                     \
    return true;                                                                   \
  }
  NSA_HEAD_DIMS(NSA_CASE)
#undef NSA_CASE
  return false;
}

}  // namespace nsa
