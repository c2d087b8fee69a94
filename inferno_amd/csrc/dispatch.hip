// Deterministic token->expert dispatch in one workgroup.
//
// Pass 1 builds the expert histogram (integer LDS atomics: the counts do not
// depend on their order), then an exclusive scan gives the expert offsets
// and the compacted list of active experts. Pass 2 is a stable scatter over
// chunks of 1024 assignments: inside a wavefront the rank of an assignment
// among earlier lanes with the same expert comes from a ballot-built match
// mask; wavefront counts per expert are prefix-summed across the 16
// wavefronts through LDS. The result equals the order of
// crates/moe/src/routing.rs:27-85 (tokens ascending, then rank), which the
// reference's GPU expert map (gguf_moe_prefill_kernels.metal:203-210, atomic
// append) does not guarantee.
#include "kernels.hpp"

namespace inferno {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxE = kMaxExperts;  // 256

__global__ void __launch_bounds__(kThreads)
    dispatch_kernel(const uint32_t* __restrict__ ids, int A, int E, uint32_t* __restrict__ offsets,
                    uint32_t* __restrict__ sorted, uint32_t* __restrict__ active) {
  __shared__ uint32_t count[kMaxE];
  __shared__ uint32_t cursor[kMaxE];
  __shared__ uint32_t wcount[kWaves * kMaxE];  // [wave][expert], row stride E
  __shared__ uint32_t scan_tmp[kThreads];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e < E; e += kThreads) count[e] = 0;
  __syncthreads();
  for (int a = tid; a < A; a += kThreads) {
    uint32_t e = ids[a];
    if (e < uint32_t(E)) atomicAdd(&count[e], 1u);
  }
  __syncthreads();
  // exclusive scan of counts (E <= 256, one value per thread)
  uint32_t c = tid < E ? count[tid] : 0u;
  scan_tmp[tid] = c;
  __syncthreads();
  for (int off = 1; off < kThreads; off <<= 1) {
    uint32_t v = tid >= off ? scan_tmp[tid - off] : 0u;
    __syncthreads();
    scan_tmp[tid] += v;
    __syncthreads();
  }
  uint32_t incl = scan_tmp[tid];
  if (tid < E) {
    offsets[tid] = incl - c;
    cursor[tid] = incl - c;
  }
  if (tid == E - 1) offsets[E] = incl;
  __syncthreads();
  // active list: the same scan over the 0/1 "has assignments" flags
  scan_tmp[tid] = (tid < E && c > 0) ? 1u : 0u;
  __syncthreads();
  for (int off = 1; off < kThreads; off <<= 1) {
    uint32_t v = tid >= off ? scan_tmp[tid - off] : 0u;
    __syncthreads();
    scan_tmp[tid] += v;
    __syncthreads();
  }
  if (tid < E && c > 0) active[scan_tmp[tid]] = uint32_t(tid);  // 1-based slot
  if (tid == kThreads - 1) active[0] = scan_tmp[tid];
  __syncthreads();

  // stable scatter
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  for (int base = 0; base < A; base += kThreads) {
    const int a = base + tid;
    const bool valid = a < A;
    const uint32_t e = valid ? ids[a] : 0xffffffffu;
    const bool ok = valid && e < uint32_t(E);
    uint64_t match = __ballot(ok);
    for (int bit = 0; bit < nbits; ++bit) {
      uint64_t b = __ballot(ok && ((e >> bit) & 1u));
      match &= ((e >> bit) & 1u) ? b : ~b;
    }
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const uint32_t rank = uint32_t(__popcll(match & lt));
    const bool leader = ok && (match & lt) == 0ull;
    // per-wave per-expert counts, written by each match group's first lane
    for (int i = tid; i < kWaves * E; i += kThreads) wcount[i] = 0u;
    __syncthreads();
    if (leader) wcount[wave * E + int(e)] = uint32_t(__popcll(match));
    __syncthreads();
    if (ok) {
      uint32_t before = 0;
      for (int w = 0; w < wave; ++w) before += wcount[w * E + int(e)];
      sorted[cursor[e] + before + rank] = uint32_t(a);
    }
    __syncthreads();
    for (int ex = tid; ex < E; ex += kThreads) {
      uint32_t tot = 0;
      for (int w = 0; w < kWaves; ++w) tot += wcount[w * E + ex];
      cursor[ex] += tot;
    }
    __syncthreads();
  }
}

}  // namespace

int launch_dispatch(hipStream_t s, const uint32_t* ids, size_t T, size_t k, size_t E,
                    uint32_t* offsets, uint32_t* sorted, uint32_t* active) {
  dispatch_kernel<<<1, kThreads, 0, s>>>(ids, int(T * k), int(E), offsets, sorted, active);
  INF_LAUNCHED();
  return INFERNO_OK;
}

}  // namespace inferno
