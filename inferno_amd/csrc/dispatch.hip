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
#include "routing_dev.hpp"

namespace inferno {
namespace {

__global__ void __launch_bounds__(kDispatchThreads)
    dispatch_kernel(const uint32_t* __restrict__ ids, int A, int E, uint32_t* __restrict__ offsets,
                    uint32_t* __restrict__ sorted, uint32_t* __restrict__ active) {
  dispatch_block(ids, A, E, offsets, sorted, active);
}

}  // namespace

int launch_dispatch(hipStream_t s, const uint32_t* ids, size_t T, size_t k, size_t E,
                    uint32_t* offsets, uint32_t* sorted, uint32_t* active) {
  dispatch_kernel<<<1, kDispatchThreads, 0, s>>>(ids, int(T * k), int(E), offsets, sorted, active);
  INF_LAUNCHED();
  return INFERNO_OK;
}

}  // namespace inferno
