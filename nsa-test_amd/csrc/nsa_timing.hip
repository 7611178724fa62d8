// Optional per-kernel timing with HIP events, recorded on the launch stream.
//
// nsa_timing_begin(id) arms event pairs around every launch of kernel `id` (ids
// below); nsa_timing_end() waits for the recorded events, returns the summed elapsed
// time and the launch count, and disarms.  When disarmed the scopes cost one branch.
#include <vector>

#include "../../include/nsa_hip.h"
#include "nsa_kernels.h"

namespace nsa {

namespace {
int g_kind = -1;
std::vector<hipEvent_t> g_start, g_stop;
size_t g_used = 0;

hipEvent_t take(std::vector<hipEvent_t>& pool, size_t i) {
  while (pool.size() <= i) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    pool.push_back(e);
  }
  return pool[i];
}
}  // namespace

TimingScope::TimingScope(int kind, hipStream_t st) : active_(kind == g_kind && kind >= 0), stream_(st) {
  if (!active_) return;
  hipEvent_t e = take(g_start, g_used);
  if (!e || !take(g_stop, g_used)) {
    active_ = false;
    return;
  }
  hipEventRecord(e, stream_);
}

TimingScope::~TimingScope() {
  if (!active_) return;
  hipEventRecord(g_stop[g_used], stream_);
  ++g_used;
}

}  // namespace nsa

extern "C" int nsa_timing_begin(int kernel_id) {
  nsa::g_kind = kernel_id;
  nsa::g_used = 0;
  return NSA_OK;
}

extern "C" int nsa_timing_end(double* total_ms, int* launches) {
  double tot = 0.0;
  for (size_t i = 0; i < nsa::g_used; ++i) {
    if (hipEventSynchronize(nsa::g_stop[i]) != hipSuccess) return nsa::set_error(NSA_ERR_HIP, "event sync failed");
    float ms = 0.f;
    hipEventElapsedTime(&ms, nsa::g_start[i], nsa::g_stop[i]);
    tot += ms;
  }
  if (total_ms) *total_ms = tot;
  if (launches) *launches = (int)nsa::g_used;
  nsa::g_kind = -1;
  nsa::g_used = 0;
  return NSA_OK;
}
