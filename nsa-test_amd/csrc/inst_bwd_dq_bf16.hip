// Instantiations: attention bwd_dq kernels, element type bf16, every (DK, DV, branch).
#include "nsa_attn_bwd_dq.h"
#include "nsa_kernels.h"

namespace nsa {

bool dispatch_attn_bwd_dq_bf16(int dk, int dv, int br, const AttnArgs& a, hipStream_t st) {
#define NSA_CASE(DKV, DVV)                                                          \
  if (dk == DKV && dv == DVV) {                                                    \
    if (br == kSliding) launch_attn_bwd_dq<bf16, DKV, DVV, kSliding>(a, st);         \
    else if (br == kCompression) launch_attn_bwd_dq<bf16, DKV, DVV, kCompression>(a, st); \
    else launch_attn_bwd_dq<bf16, DKV, DVV, kSelection>(a, st);                     \
    return true;                                                                   \
  }
  NSA_HEAD_DIMS(NSA_CASE)
#undef NSA_CASE
  return false;
}

}  // namespace nsa
