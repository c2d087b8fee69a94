// RMSNorm -> router logits (-> exact top-k) of decode tokens in one launch.
//
// Reference: laguna_xs_rms_norm_router_decode_f32_kernel
// (crates/backend/src/metal/kernels/laguna_xs_kernels.metal:1274-1365,
// trait method Backend::laguna_xs_rms_norm_router_device,
// crates/backend/src/backend.rs:1162): every threadgroup recomputes the small
// normalisation of the token's row, keeps it in threadgroup memory and owns
// a few router rows; threadgroup zero publishes the normalised row. The top-k
// that follows there in its own launch (laguna_xs_router_top8_decode_f32_kernel,
// :1077-1165; semantics crates/model/src/moe_router.rs:835-936) runs here in
// the same launch, in the last workgroup of the token to finish its logits.
//
// Workgroup (g, t), 1024 threads: rms_norm_row (the RMSNorm launch's own
// code, so the normalised row is bit-identical to it) into LDS, rounded to
// the activation type the experts take (fp32 or bf16); then expert g, its
// 16 wavefronts over a sixteenth of H each (float4 lanes, wave butterfly,
// parts added in order): fixed order, no float atomics. With
// the top-k: the logits go to the workspace, each workgroup releases them
// (agent-scope fence) and takes a ticket; the one that draws the last ticket
// acquires, reads the token's E logits and selects on one wavefront
// (topk_row_wave, the router entry point's selection), then puts the ticket
// back to zero for the next call. No workgroup waits for another.
#include "kernels.hpp"
#include "norm_dev.hpp"
#include "routing_dev.hpp"

namespace inferno {
namespace {

constexpr int kNrExperts = 1;  // experts per workgroup
constexpr int kNrParts = 16 / kNrExperts;  // wavefronts (H parts) per expert
constexpr int kNrMaxH = 8192;  // LDS row of fp32 values (32 KB)

struct NormRouterArgs {
  const float* x;        // [T, H] fp32 rows (the residual stream)
  const float* norm_w;   // [H]
  const float* router;   // [E, H] fp32
  const float* bias;     // [E] or null (top-k only)
  int T, H, E, k, score_fn, norm, act_dtype;
  float eps, scale;
  void* normed;          // [T, H] act_dtype, or null
  float* logits;         // [T, E]
  uint32_t* tickets;     // [T], zero on entry, left zero (top-k only)
  uint32_t* ids;         // [T, k] (null: no top-k)
  float* weights;        // [T, k]
};

__global__ void __launch_bounds__(kNormThreads) norm_router_kernel(NormRouterArgs a) {
  __shared__ float xn[kNrMaxH];
  __shared__ float part[kNormThreads / 64 + 1];
  __shared__ float lp[kNrParts][kNrExperts];
  __shared__ uint32_t last;
  __shared__ float row[kMaxExperts];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t = blockIdx.y, H = a.H, E = a.E;
  const bool bf16 = a.act_dtype == INFERNO_BF16;
  const bool publish = blockIdx.x == 0 && a.normed != nullptr;
  rms_norm_row(a.x + size_t(t) * H, a.norm_w, size_t(H), a.eps, part, [&](size_t i, float v) {
    if (bf16) {
      const uint16_t b = f32_to_bf16_bits(v);
      xn[i] = bf16_bits_to_f32(b);
      if (publish) static_cast<uint16_t*>(a.normed)[size_t(t) * H + i] = b;
    } else {
      xn[i] = v;
      if (publish) static_cast<float*>(a.normed)[size_t(t) * H + i] = v;
    }
  });
  __syncthreads();
  // expert e0 + (wave % kNrExperts) over part (wave / kNrExperts) of H
  const int el = wave % kNrExperts, qh = wave / kNrExperts, e = int(blockIdx.x) * kNrExperts + el;
  const int q4 = H / (4 * kNrParts);  // float4s per part
  float acc = 0.f;
  if (e < E) {
    const float4* w4 = reinterpret_cast<const float4*>(a.router + size_t(e) * H) + qh * q4;
    const float4* x4 = reinterpret_cast<const float4*>(xn) + qh * q4;
    for (int i = lane; i < q4; i += kWave) {
      const float4 w = w4[i], x = x4[i];
      acc = fmaf(x.x, w.x, acc);
      acc = fmaf(x.y, w.y, acc);
      acc = fmaf(x.z, w.z, acc);
      acc = fmaf(x.w, w.w, acc);
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) lp[qh][el] = acc;
  __syncthreads();
  if (tid < kNrExperts) {
    const int ee = int(blockIdx.x) * kNrExperts + tid;
    float v = 0.f;
#pragma unroll
    for (int j = 0; j < kNrParts; ++j) v += lp[j][tid];
    if (ee < E) a.logits[size_t(t) * E + ee] = v;
  }
  if (a.ids == nullptr) return;  // uniform
  if (tid == 0) {
    // the logits this workgroup wrote (thread 0's own stores) reach device
    // scope before its ticket; the last ticket holder sees every logit
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const uint32_t old = __hip_atomic_fetch_add(a.tickets + t, 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    last = old == gridDim.x - 1 ? 1u : 0u;
  }
  __syncthreads();
  if (!last) return;  // uniform
  if (tid == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  __syncthreads();
  for (int i = tid; i < E; i += kNormThreads)
    row[i] = __hip_atomic_load(a.logits + size_t(t) * E + i, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (wave == 0) {
    uint32_t sel[kMaxTopK];
    topk_row_wave(row, a.bias, E, a.k, a.score_fn, a.norm, a.scale, t, a.ids, a.weights, nullptr,
                  sel);
    if (lane == 0)
      __hip_atomic_store(a.tickets + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace

bool norm_router_supported(size_t T, size_t H, size_t E, size_t k) {
  return T >= 1 && T <= 65535 && H % (4 * kNrParts) == 0 && H >= 4 * kNrParts && H <= size_t(kNrMaxH) && E >= 1 &&
         E <= size_t(kMaxExperts) && k <= E && k <= size_t(kMaxTopK);
}

int launch_norm_router(hipStream_t s, const float* x, const float* norm_w, float eps,
                       const float* router, const float* bias, size_t T, size_t H, size_t E,
                       size_t k, int score_fn, int norm, float scale, int act_dtype, void* normed,
                       float* logits, uint32_t* tickets, uint32_t* ids, float* weights) {
  if (T == 0) return INFERNO_OK;
  NormRouterArgs a{};
  a.x = x; a.norm_w = norm_w; a.router = router; a.bias = bias;
  a.T = int(T); a.H = int(H); a.E = int(E); a.k = int(k);
  a.score_fn = score_fn; a.norm = norm; a.act_dtype = act_dtype;
  a.eps = eps; a.scale = scale;
  a.normed = normed; a.logits = logits; a.tickets = tickets; a.ids = ids; a.weights = weights;
  const dim3 grid(unsigned((E + kNrExperts - 1) / kNrExperts), unsigned(T));
  norm_router_kernel<<<grid, kNormThreads, 0, s>>>(a);
  INF_LAUNCHED();
  return INFERNO_OK;
}

}  // namespace inferno
