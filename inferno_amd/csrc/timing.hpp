// Measurement hook: HIP events around the routed expert launches, summed per
// timer while enabled (inferno_kernel_timing_* in the C ABI).
#pragma once
#include "common.hpp"

namespace inferno {

enum KernelTimer { kTimerGateUp = 0, kTimerDown = 1, kTimerRoute = 2, kTimerSelect = 3, kNumTimers = 4 };

void kernel_timing_enable(bool on);
// Sums the timer's recorded launches (waiting for them) and resets it.
bool kernel_timing_read(int which, double* ms, uint64_t* n);
bool kernel_timing_on();
// An event pair of the current device for one timed launch (pooled).
int kernel_timing_begin(hipEvent_t* start, hipEvent_t* stop, int* dev);
// Returns a pair taken by kernel_timing_begin whose launch failed to the pool.
void kernel_timing_abort(int dev, hipEvent_t start, hipEvent_t stop);
// Files the recorded pair under timer `which`; read sums it later.
void kernel_timing_end(int which, int dev, hipEvent_t start, hipEvent_t stop, const char* label);
// Label of the last launch a timer measured (a static string), or "".
const char* kernel_timing_label(int which);

// Runs `launch` (returns a status) on stream s; when timing is on, brackets
// it with events recorded without waiting (the elapsed times are summed when
// the timer is read). `label` (a static string) names what the launch
// covers; the bench reads it back to know which bytes the launch streamed.
template <typename Fn>
int timed(hipStream_t s, int which, const char* label, Fn launch) {
  if (!kernel_timing_on()) return launch();
  hipEvent_t e0, e1;
  int dev = 0, st;
  if ((st = kernel_timing_begin(&e0, &e1, &dev))) return st;
  hipError_t e = hipEventRecord(e0, s);
  if (e == hipSuccess) {
    if ((st = launch())) {
      kernel_timing_abort(dev, e0, e1);
      return st;
    }
    e = hipEventRecord(e1, s);
  }
  if (e != hipSuccess) {
    kernel_timing_abort(dev, e0, e1);
    set_error(std::string("hipEventRecord: ") + hipGetErrorString(e));
    return INFERNO_ERR_DEVICE;
  }
  kernel_timing_end(which, dev, e0, e1, label);
  return INFERNO_OK;
}

}  // namespace inferno
