// Deterministic token->expert dispatch (one workgroup, or one per chunk of
// 2048 assignments for large batches).
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
#include "routing_dev.hpp"

namespace inferno {
namespace {

__global__ void __launch_bounds__(kDispatchThreads)
    dispatch_kernel(const uint32_t* __restrict__ ids, int A, int E, uint32_t* __restrict__ offsets,
                    uint32_t* __restrict__ sorted, uint32_t* __restrict__ active, PlanOut plan) {
  dispatch_block(ids, A, E, offsets, sorted, active, plan);
}

// Many assignments: workgroup b scatters chunk [b kChunk, (b + 1) kChunk).
// Each workgroup histograms all assignments itself (per-wavefront counts of
// match groups, no atomics), split into those before
// its chunk and the total, so its cursors are offsets[e] + (assignments of e
// before the chunk) and the result is the single-workgroup order; no
// workspace and no cross-workgroup synchronisation. Workgroup 0 writes the
// offsets and the active list.
constexpr int kChunk = 2 * kDispatchThreads;

__global__ void __launch_bounds__(kDispatchThreads)
    dispatch_chunks_kernel(const uint32_t* __restrict__ ids, int A, int E,
                           uint32_t* __restrict__ offsets, uint32_t* __restrict__ sorted,
                           uint32_t* __restrict__ active, PlanOut plan) {
  __shared__ uint32_t total[kMaxExperts], before[kMaxExperts], cursor[kMaxExperts];
  // per-wavefront counts (rows of wcount: totals, of wbefore: before the
  // chunk): a match group's leader is the only writer of its expert's slot
  // in its own row, so no atomics; rows are summed afterwards
  __shared__ uint32_t wcount[kDispatchWaves * kMaxExperts];
  __shared__ uint32_t wbefore[kDispatchWaves * kMaxExperts];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int a0 = int(blockIdx.x) * kChunk;
  const int nbits = expert_bits(E);
  for (int i = tid; i < kDispatchWaves * E; i += kDispatchThreads) wcount[i] = wbefore[i] = 0u;
  __syncthreads();
  uint32_t* wt = wcount + wave * E;
  uint32_t* wb = wbefore + wave * E;
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  constexpr int U = 8;  // ids loaded ahead per thread
  for (int base = 0; base < A; base += U * kDispatchThreads) {
    uint32_t ev[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int a = base + u * kDispatchThreads + tid;
      const uint32_t id = ids[min(a, A - 1)];  // clamped: the U loads go out together
      ev[u] = a < A ? id : 0xffffffffu;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = base + u * kDispatchThreads;
      const uint32_t e = ev[u];
      const bool ok = e < uint32_t(E);
      const uint64_t match = expert_match(e, ok, nbits);
      if (ok && (match & lt) == 0ull) {
        const uint32_t n = uint32_t(__popcll(match));
        wt[e] += n;
        if (b < a0) wb[e] += n;  // a0 is a multiple of 1024
      }
    }
  }
  __syncthreads();
  for (int e = tid; e < E; e += kDispatchThreads) {
    uint32_t t = 0, b = 0;
    for (int w = 0; w < kDispatchWaves; ++w) {
      t += wcount[w * E + e];
      b += wbefore[w * E + e];
    }
    total[e] = t;
    before[e] = b;
  }
  __syncthreads();
  if (wave == 0) dispatch_scan(total, E, cursor, blockIdx.x == 0, offsets, active, plan);
  __syncthreads();
  for (int e = tid; e < E; e += kDispatchThreads) cursor[e] += before[e];
  __syncthreads();
  dispatch_scatter(ids, a0, min(a0 + kChunk, A), E, cursor, wcount, sorted);
}

}  // namespace

int launch_dispatch(hipStream_t s, const uint32_t* ids, size_t T, size_t k, size_t E,
                    uint32_t* offsets, uint32_t* sorted, uint32_t* active, const PlanOut* plan) {
  const size_t A = T * k;
  const PlanOut po = plan ? *plan : PlanOut{};
  if (A > size_t(2 * kChunk))
    dispatch_chunks_kernel<<<unsigned((A + kChunk - 1) / kChunk), kDispatchThreads, 0, s>>>(
        ids, int(A), int(E), offsets, sorted, active, po);
  else
    dispatch_kernel<<<1, kDispatchThreads, 0, s>>>(ids, int(A), int(E), offsets, sorted, active,
                                                   po);
  INF_LAUNCHED();
  return INFERNO_OK;
}

}  // namespace inferno
