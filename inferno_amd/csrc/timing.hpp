// Measurement hook: HIP events around the routed expert launches, summed per
// timer while enabled (inferno_kernel_timing_* in the C ABI).
#pragma once
#include "common.hpp"

namespace inferno {

enum KernelTimer { kTimerGateUp = 0, kTimerDown = 1, kTimerRoute = 2, kTimerSelect = 3, kNumTimers = 4 };

void kernel_timing_enable(bool on);
bool kernel_timing_read(int which, double* ms, uint64_t* n);
bool kernel_timing_on();
// Start/stop events of the current device (created on first use).
int kernel_timing_events(hipEvent_t* start, hipEvent_t* stop);
void kernel_timing_add(int which, float ms, const char* label);
// Label of the last launch a timer measured (a static string), or "".
const char* kernel_timing_label(int which);

// Runs `launch` (returns a status) on stream s; when timing is on, brackets
// it with events, waits for the stop event and adds the elapsed time.
// `label` (a static string) names what the launch covers; the bench reads
// it back to know which bytes the timed launch streamed.
template <typename Fn>
int timed(hipStream_t s, int which, const char* label, Fn launch) {
  if (!kernel_timing_on()) return launch();
  hipEvent_t e0, e1;
  int st;
  if ((st = kernel_timing_events(&e0, &e1))) return st;
  INF_HIP(hipEventRecord(e0, s));
  if ((st = launch())) return st;
  INF_HIP(hipEventRecord(e1, s));
  INF_HIP(hipEventSynchronize(e1));
  float ms = 0.f;
  INF_HIP(hipEventElapsedTime(&ms, e0, e1));
  kernel_timing_add(which, ms, label);
  return INFERNO_OK;
}

}  // namespace inferno
