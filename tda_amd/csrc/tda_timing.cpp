// tda_timing.cpp -- per-launch timing of one C-ABI call (tda_time_next_call): the caller's
// events are recorded on the call's stream before the first kernel launch and after each
// launch, so the caller reads every kernel's duration with hipEventElapsedTime on the stream
// the kernels ran on.  No counterpart in the reference.  State is per host thread and covers
// one call: the launchers report each launch through tda::launched().
#include <hip/hip_runtime_api.h>

#include "../../include/tda.h"
#include "tda_params.hpp"

namespace {

constexpr int kMaxNamed = 16;

struct Timing {
  void* const* ev = nullptr;  // armed: the events of the next call
  int n = 0;
  bool active = false;        // inside the timed call
  int recorded = 0;           // events recorded in the current call
  int launches = 0;           // launches of the current (or last timed) call
  int error = 0;              // first failed event record (hipError_t)
  const char* names[kMaxNamed] = {};
};
thread_local Timing g_t;

void record(hipStream_t s) {
  if (g_t.recorded >= g_t.n) return;
  const hipError_t e = hipEventRecord((hipEvent_t)g_t.ev[g_t.recorded], s);
  if (e != hipSuccess && !g_t.error) g_t.error = (int)e;
  ++g_t.recorded;
}

}  // namespace

namespace tda {

void timing_begin(void* stream) {
  if (!g_t.ev || g_t.n <= 0) return;
  g_t.active = true;
  g_t.recorded = g_t.launches = g_t.error = 0;
  record((hipStream_t)stream);
}

void launched(void* stream, const char* name) {
  if (!g_t.active) return;
  if (g_t.launches < kMaxNamed) g_t.names[g_t.launches] = name;
  ++g_t.launches;
  record((hipStream_t)stream);
}

int timing_end() {
  if (!g_t.active) return 0;
  g_t.active = false;
  g_t.ev = nullptr;
  g_t.n = 0;
  return g_t.error;
}

}  // namespace tda

extern "C" {

int32_t tda_time_next_call(void* const* events, int32_t n) {
  if (n > 0 && !events) return TDA_ERR_NULL_POINTER;
  g_t.ev = n > 0 ? events : nullptr;
  g_t.n = n > 0 ? n : 0;
  return TDA_OK;
}

int32_t tda_timed_launches(void) { return g_t.launches; }

const char* tda_timed_launch_name(int32_t k) {
  return (k >= 0 && k < g_t.launches && k < kMaxNamed) ? g_t.names[k] : nullptr;
}

}  // extern "C"
