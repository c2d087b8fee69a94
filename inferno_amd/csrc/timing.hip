// Process-wide state of the kernel timing hook.
#include "timing.hpp"

#include <mutex>
#include <vector>

namespace inferno {
namespace {

// Event pairs are recorded around the timed launches without waiting (a
// wait per launch would start every kernel on an idle device and add the
// launch latency to its time); the pairs are summed when a timer is read.
struct Pending {
  int which, dev;
  hipEvent_t e0, e1;
};

struct KernelTimers {
  std::mutex mu;
  bool on = false;
  double ms[kNumTimers] = {};
  uint64_t n[kNumTimers] = {};
  const char* label[kNumTimers] = {};
  std::vector<Pending> pending;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> free_pairs[64];
};

KernelTimers& timers() {
  static KernelTimers t;
  return t;
}

}  // namespace

void kernel_timing_enable(bool on) {
  std::lock_guard<std::mutex> lock(timers().mu);
  KernelTimers& k = timers();
  k.on = on;
  if (!on) {
    // timing off: unread launches are dropped (after they complete, so the
    // pairs can be recorded again) and the sums cleared
    for (const Pending& pd : k.pending) {
      (void)hipEventSynchronize(pd.e1);
      k.free_pairs[pd.dev].push_back({pd.e0, pd.e1});
    }
    k.pending.clear();
    for (int i = 0; i < kNumTimers; ++i) {
      k.ms[i] = 0;
      k.n[i] = 0;
    }
  }
}

bool kernel_timing_on() {
  std::lock_guard<std::mutex> lock(timers().mu);
  return timers().on;
}

bool kernel_timing_read(int which, double* ms, uint64_t* n) {
  if (which < 0 || which >= kNumTimers) return false;
  std::lock_guard<std::mutex> lock(timers().mu);
  KernelTimers& k = timers();
  // settle this timer's pending pairs (in recording order)
  std::vector<Pending> keep;
  for (const Pending& pd : k.pending) {
    if (pd.which != which) {
      keep.push_back(pd);
      continue;
    }
    float t = 0.f;
    if (hipEventSynchronize(pd.e1) == hipSuccess && hipEventElapsedTime(&t, pd.e0, pd.e1) == hipSuccess) {
      k.ms[which] += t;
      k.n[which] += 1;
    }
    k.free_pairs[pd.dev].push_back({pd.e0, pd.e1});
  }
  k.pending.swap(keep);
  *ms = k.ms[which];
  *n = k.n[which];
  k.ms[which] = 0;
  k.n[which] = 0;
  return true;
}

int kernel_timing_begin(hipEvent_t* start, hipEvent_t* stop, int* dev_out) {
  int dev = 0;
  INF_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) {
    set_error("device index out of range");
    return INFERNO_ERR_DEVICE;
  }
  std::lock_guard<std::mutex> lock(timers().mu);
  auto& fp = timers().free_pairs[dev];
  if (fp.empty()) {
    hipEvent_t a, b;
    // no system-scope fence when an event completes (an L2 write-back per
    // event that the timing does not need: the events only timestamp
    // kernels of one stream)
    INF_HIP(hipEventCreateWithFlags(&a, hipEventDisableSystemFence));
    const hipError_t e = hipEventCreateWithFlags(&b, hipEventDisableSystemFence);
    if (e != hipSuccess) {
      (void)hipEventDestroy(a);
      set_error(std::string("hipEventCreateWithFlags: ") + hipGetErrorString(e));
      return INFERNO_ERR_DEVICE;
    }
    fp.push_back({a, b});
  }
  *start = fp.back().first;
  *stop = fp.back().second;
  fp.pop_back();
  *dev_out = dev;
  return INFERNO_OK;
}

void kernel_timing_end(int which, int dev, hipEvent_t start, hipEvent_t stop, const char* label) {
  std::lock_guard<std::mutex> lock(timers().mu);
  timers().pending.push_back({which, dev, start, stop});
  timers().label[which] = label;
}

void kernel_timing_abort(int dev, hipEvent_t start, hipEvent_t stop) {
  std::lock_guard<std::mutex> lock(timers().mu);
  timers().free_pairs[dev].push_back({start, stop});
}

const char* kernel_timing_label(int which) {
  if (which < 0 || which >= kNumTimers) return "";
  std::lock_guard<std::mutex> lock(timers().mu);
  return timers().label[which] ? timers().label[which] : "";
}

}  // namespace inferno
