// Process-wide state of the kernel timing hook.
#include "timing.hpp"

#include <mutex>

namespace inferno {
namespace {

struct KernelTimers {
  std::mutex mu;
  bool on = false;
  double ms[kNumTimers] = {};
  uint64_t n[kNumTimers] = {};
  const char* label[kNumTimers] = {};
  hipEvent_t ev[64][2] = {};
};

KernelTimers& timers() {
  static KernelTimers t;
  return t;
}

}  // namespace

void kernel_timing_enable(bool on) {
  std::lock_guard<std::mutex> lock(timers().mu);
  timers().on = on;
}

bool kernel_timing_on() {
  std::lock_guard<std::mutex> lock(timers().mu);
  return timers().on;
}

bool kernel_timing_read(int which, double* ms, uint64_t* n) {
  if (which < 0 || which >= kNumTimers) return false;
  std::lock_guard<std::mutex> lock(timers().mu);
  *ms = timers().ms[which];
  *n = timers().n[which];
  timers().ms[which] = 0;
  timers().n[which] = 0;
  return true;
}

int kernel_timing_events(hipEvent_t* start, hipEvent_t* stop) {
  int dev = 0;
  INF_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) {
    set_error("device index out of range");
    return INFERNO_ERR_DEVICE;
  }
  std::lock_guard<std::mutex> lock(timers().mu);
  hipEvent_t* ev = timers().ev[dev];
  if (!ev[0]) {
    INF_HIP(hipEventCreate(&ev[0]));
    INF_HIP(hipEventCreate(&ev[1]));
  }
  *start = ev[0];
  *stop = ev[1];
  return INFERNO_OK;
}

void kernel_timing_add(int which, float ms, const char* label) {
  std::lock_guard<std::mutex> lock(timers().mu);
  timers().ms[which] += ms;
  timers().n[which] += 1;
  timers().label[which] = label;
}

const char* kernel_timing_label(int which) {
  if (which < 0 || which >= kNumTimers) return "";
  std::lock_guard<std::mutex> lock(timers().mu);
  return timers().label[which] ? timers().label[which] : "";
}

}  // namespace inferno
