// Fused decode path of one MoE layer (T <= 64 tokens), five launches on the
// layer's stream plus two on a side stream:
//
//   route    router logits as per-chunk partial sums (H split over many
//            workgroups) + staging of x into packed-f16 runs;
//   select   logits = ordered sum of the partials, exact top-k per token
//            (one wavefront each), stable dispatch (one wavefront for T = 1);
//   gate/up  routed 16-row tiles, writing the SwiGLU intermediate already
//            staged for the down pass;
//   down     routed 16-row tiles, one output row per assignment;
//   combine  out = residual + shared + sum over ranks in rank order,
//            deterministic without float atomics.
// The Q8_0 shared expert (gate/up + down) only needs the staged x and runs
// on the side stream between route and combine.
//
// Reference semantics: crates/model/src/laguna/gguf_model.rs:731-860 (layer
// order), gguf_moe_kernels.metal:340-565 (routed SwiGLU with the routing
// weight folded, down summed over ranks), q2_kernels.metal:2066-2235
// (shared expert plus two residual adds), moe_kernels.metal:210-238 (rank
// order combine).
#include "decode.hpp"
#include "dot2_formats.hpp"
#include "routing_dev.hpp"

#include <mutex>

namespace inferno {
namespace {

constexpr int kMaxDecodeTokens = 64;

// ------------------------------------------------------------------ route

template <typename XT>
__global__ void __launch_bounds__(256) route_kernel(DecodeArgs p) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int T = p.T, H = p.H, E = p.E;
  // staging: one thread per 16-value run of x
  {
    const int g = blockIdx.x + blockIdx.y * gridDim.x;
    const int run_id = g * 256 + tid;
    const int runs = H / 16;
    if (run_id < T * runs) {
      const int t = run_id / runs, run = run_id % runs;
      const XT* src = static_cast<const XT*>(p.x) + size_t(t) * H + run * 16;
      float v[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = to_f32(src[i]);
      constexpr bool kSplit = !std::is_same<XT, uint16_t>::value;
      stage_run<kSplit>(v, p.stage_x + size_t(t) * staged_stride(H, kSplit), H, run);
    }
  }
  // logits partial of expert e over chunk c for every token
  const int e = blockIdx.x * 4 + wave;
  const int c = blockIdx.y;
  if (e >= E || c >= p.n_chunks) return;
  const int h0 = c * p.chunk;
  const float* wrow = p.router + size_t(e) * H + h0;
  float acc[16];
  for (int t0 = 0; t0 < T; t0 += 16) {
#pragma unroll
    for (int t = 0; t < 16; ++t) acc[t] = 0.f;
    for (int i = lane * 4; i < p.chunk; i += 256) {
      const float4 wv = *reinterpret_cast<const float4*>(wrow + i);
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        if (t0 + t < T) {
          const XT* xr = static_cast<const XT*>(p.x) + size_t(t0 + t) * H + h0 + i;
          acc[t] += wv.x * to_f32(xr[0]) + wv.y * to_f32(xr[1]) + wv.z * to_f32(xr[2]) +
                    wv.w * to_f32(xr[3]);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      if (t0 + t < T) {
        const float s = wave_sum(acc[t]);
        if (lane == 0) p.partials[(size_t(c) * T + t0 + t) * E + e] = s;
      }
    }
  }
}

// ----------------------------------------------------------------- select

// T = 1: one wavefront does everything. The k selected ids are distinct,
// so the dispatch is the k ids sorted ascending (one assignment each).
__global__ void __launch_bounds__(64) select1_kernel(DecodeArgs p) {
  __shared__ float logit_row[kMaxExperts];
  const int lane = threadIdx.x;
  const int E = p.E, k = p.k;
  for (int e = lane; e < E; e += 64) {
    float s = 0.f;
    for (int c = 0; c < p.n_chunks; ++c) s += p.partials[size_t(c) * E + e];
    logit_row[e] = s;
  }
  __builtin_amdgcn_wave_barrier();  // LDS is in order within a wavefront
  uint32_t all[kMaxTopK];  // the k selected ids, held by every lane
  topk_row_wave(logit_row, p.bias, E, k, p.score_fn, p.norm, p.scale, 0, p.ids, p.weights,
                nullptr, all);
  uint32_t id = 0xffffffffu;
#pragma unroll
  for (int j = 0; j < kMaxTopK; ++j)
    if (j == lane) id = all[j];
  // rank of each id among the k (distinct) ids
  uint32_t rank = 0;
#pragma unroll
  for (int j = 0; j < kMaxTopK; ++j) rank += (j < k && all[j] < id) ? 1u : 0u;
  if (lane < k) {
    p.sorted[rank] = uint32_t(lane);  // assignment index t*k + r with t = 0
    p.active[1 + rank] = id;
  }
  if (lane == 0) p.active[0] = uint32_t(k);
  // offsets[e] = number of ids below e
  for (int e = lane; e <= E; e += 64) {
    uint32_t below = 0;
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) below += (j < k && all[j] < uint32_t(e)) ? 1u : 0u;
    p.offsets[e] = below;
  }
}

__global__ void __launch_bounds__(1024) select_kernel(DecodeArgs p) {
  __shared__ float logit_row[16][kMaxExperts];
  __shared__ uint32_t ids_lds[kMaxDecodeTokens * kMaxTopK];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int T = p.T, E = p.E, k = p.k;
  for (int t = wave; t < T; t += 16) {
    for (int e = lane; e < E; e += 64) {
      float s = 0.f;
      for (int c = 0; c < p.n_chunks; ++c) s += p.partials[(size_t(c) * T + t) * E + e];
      logit_row[wave][e] = s;
    }
    __builtin_amdgcn_wave_barrier();  // LDS is in order within a wavefront
    uint32_t sel[kMaxTopK];
    topk_row_wave(logit_row[wave], p.bias, E, k, p.score_fn, p.norm, p.scale, t, p.ids,
                  p.weights, nullptr, sel);
#pragma unroll
    for (int r = 0; r < kMaxTopK; ++r)
      if (r < k && lane == r) ids_lds[t * k + r] = sel[r];
  }
  __syncthreads();
  dispatch_block(ids_lds, T * k, E, p.offsets, p.sorted, p.active);
}

// ---------------------------------------------------------------- experts

//
// Grid launches over 16-row tiles, ordered by the stream only: no workgroup
// waits for or signals another inside a launch. (On this multi-XCD part an
// agent-scope fence is an L2-wide writeback or invalidate, far too costly
// per tile, and spinning on another workgroup's progress cannot be bounded.)

// gate/up: routed grid = max_slots * tiles_i tiles (slot = tile / tiles_i,
// idle when slot >= active[0]); shared grid = tiles_is tiles of the Q8_0
// shared expert. The two run as separate launches on two streams.
template <int Q, bool XSPLIT, bool SHARED>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 8)))
    gate_up_kernel(DecodeArgs p) {
  extern __shared__ uint32_t smem[];
  const int tid = threadIdx.x, slot = (tid & 63) >> 2;
  const int T = p.T, H = p.H, I = p.I, Is = p.Is, k = p.k;
  const int Sx = staged_stride(H, XSPLIT);
  const int tiles_i = I / kRows;
  const uint32_t item = blockIdx.x;
  constexpr bool shared = SHARED;
  const uint32_t j = shared ? 0u : item / uint32_t(tiles_i);
  if (!shared && j >= p.active[0]) return;
  const int tile = shared ? int(item) : int(item % uint32_t(tiles_i));
  const int row = tile * kRows + slot;
  uint32_t* xs = smem;
  float* part = reinterpret_cast<float*>(smem + Sx);
  float* res = part + tile_part_floats(1);
  uint32_t lo = 0, hi = uint32_t(T);
  const uint8_t *r0, *r1;
  const size_t rb = size_t(H / kKBlock) * Fmt<Q>::kBytes;
  if constexpr (!shared) {
    const uint32_t e = p.active[1 + j];
    lo = p.offsets[e];
    hi = p.offsets[e + 1];
    r0 = p.gate + size_t(e) * p.gate_stride + size_t(row) * rb;
    r1 = p.up + size_t(e) * p.gate_stride + size_t(row) * rb;
  } else {
    r0 = p.sgate + size_t(row) * rb;
    r1 = p.sup + size_t(row) * rb;
  }
  for (uint32_t c = lo; c < hi; ++c) {
    const uint32_t a = shared ? c : p.sorted[c];
    const uint32_t tok = shared ? c : a / uint32_t(k);
    copy_rows_to_lds(xs, Sx, 1, [&](int) { return p.stage_x + size_t(tok) * Sx; });
    __syncthreads();
    tile_dot<Q, 2, 1, XSPLIT>(r0, r1, H, xs, Sx, 1, part, res);
    if (tid < 16) {
      if constexpr (!shared)
        swiglu_tile_out(res, 1, 0, p.weights[a], nullptr,
                        p.stage_h + size_t(a) * staged_stride(I, true), I, tile);
      else
        swiglu_tile_out(res, 1, 0, 1.0f, nullptr,
                        p.stage_hs + size_t(c) * staged_stride(Is, true), Is, tile);
    }
    __syncthreads();
  }
}

// down: routed grid = max_slots * tiles_h tiles writing rows of y (per
// assignment); shared grid = tiles_h tiles writing rows of ys.
template <int Q, bool SHARED>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 8)))
    down_kernel(DecodeArgs p) {
  extern __shared__ uint32_t smem[];
  const int tid = threadIdx.x, slot = (tid & 63) >> 2;
  const int T = p.T, H = p.H, I = p.I, Is = p.Is;
  const int tiles_h = H / kRows;
  const uint32_t item = blockIdx.x;
  constexpr bool shared = SHARED;
  const uint32_t j = shared ? 0u : item / uint32_t(tiles_h);
  if (!shared && j >= p.active[0]) return;
  const int tile = shared ? int(item) : int(item % uint32_t(tiles_h));
  const int row = tile * kRows + slot;
  const int K = shared ? Is : I;
  const int S = staged_stride(K, true);
  uint32_t* xs = smem;
  float* part = reinterpret_cast<float*>(smem + S);  // after the staged row
  float* res = part + tile_part_floats(1);
  uint32_t lo = 0, hi = uint32_t(T);
  const uint8_t* r0;
  if constexpr (!shared) {
    const uint32_t e = p.active[1 + j];
    lo = p.offsets[e];
    hi = p.offsets[e + 1];
    r0 = p.down + size_t(e) * p.down_stride + size_t(row) * size_t(I / kKBlock) * Fmt<Q>::kBytes;
  } else {
    r0 = p.sdown + size_t(row) * size_t(Is / kKBlock) * Fmt<Q>::kBytes;
  }
  for (uint32_t c = lo; c < hi; ++c) {
    const uint32_t orow = shared ? c : p.sorted[c];
    copy_rows_to_lds(xs, S, 1, [&](int) {
      return shared ? p.stage_hs + size_t(c) * S : p.stage_h + size_t(orow) * S;
    });
    __syncthreads();
    tile_dot<Q, 1, 1, true>(r0, nullptr, K, xs, S, 1, part, res);
    if (tid < kRows) (shared ? p.ys : p.y)[size_t(orow) * H + tile * kRows + tid] = res[tid];
    __syncthreads();
  }
}

// out = residual + ys + sum over ranks of y (rank order): one thread per output.
__global__ void __launch_bounds__(256) combine_kernel(DecodeArgs p) {
  const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= size_t(p.T) * p.H) return;
  const size_t t = i / p.H, r = i % p.H;
  float y[kMaxTopK];
#pragma unroll
  for (int rk = 0; rk < kMaxTopK; ++rk)
    y[rk] = rk < p.k ? p.y[(t * p.k + rk) * p.H + r] : 0.f;
  float v = (p.residual ? p.residual[i] : 0.f) + (p.Is ? p.ys[i] : 0.f);
#pragma unroll
  for (int rk = 0; rk < kMaxTopK; ++rk)
    if (rk < p.k) v += y[rk];
  p.out[i] = v;
}

template <int Q, bool XSPLIT>
int launch_routed(hipStream_t s, const DecodeArgs& a) {
  const size_t gu_tiles = size_t(a.max_slots) * (a.I / kRows);
  const size_t gu_lds = (size_t(staged_stride(a.H, XSPLIT)) + tile_part_floats(1) + 2 * kRows) * 4;
  gate_up_kernel<Q, XSPLIT, false><<<unsigned(gu_tiles), 256, gu_lds, s>>>(a);
  INF_LAUNCHED();
  const size_t dn_tiles = size_t(a.max_slots) * (a.H / kRows);
  const size_t dn_lds = (size_t(staged_stride(a.I, true)) + tile_part_floats(1) + 2 * kRows) * 4;
  down_kernel<Q, false><<<unsigned(dn_tiles), 256, dn_lds, s>>>(a);
  INF_LAUNCHED();
  return INFERNO_OK;
}

template <bool XSPLIT>
int launch_shared(hipStream_t s, const DecodeArgs& a) {
  const size_t gu_lds = (size_t(staged_stride(a.H, XSPLIT)) + tile_part_floats(1) + 2 * kRows) * 4;
  gate_up_kernel<INFERNO_Q8_0, XSPLIT, true><<<unsigned(a.Is / kRows), 256, gu_lds, s>>>(a);
  INF_LAUNCHED();
  const size_t dn_lds = (size_t(staged_stride(a.Is, true)) + tile_part_floats(1) + 2 * kRows) * 4;
  down_kernel<INFERNO_Q8_0, true><<<unsigned(a.H / kRows), 256, dn_lds, s>>>(a);
  INF_LAUNCHED();
  return INFERNO_OK;
}

// Second stream per device for the shared expert, plus the two events of
// the fork/join. Created once, default priority, never destroyed.
struct SideStream {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};

int side_stream(SideStream** out) {
  static std::mutex mu;
  static SideStream per_device[64];
  int dev = 0;
  INF_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) {
    set_error("device index out of range");
    return INFERNO_ERR_DEVICE;
  }
  std::lock_guard<std::mutex> lock(mu);
  SideStream& ss = per_device[dev];
  if (!ss.stream) {
    INF_HIP(hipStreamCreateWithFlags(&ss.stream, hipStreamNonBlocking));
    INF_HIP(hipEventCreateWithFlags(&ss.fork, hipEventDisableTiming));
    INF_HIP(hipEventCreateWithFlags(&ss.join, hipEventDisableTiming));
  }
  *out = &ss;
  return INFERNO_OK;
}

}  // namespace

bool decode_supported(size_t T, size_t k, size_t E, int quant, int down_quant) {
  return T >= 1 && T <= size_t(kMaxDecodeTokens) && T * k <= size_t(kMaxDecodeTokens * kMaxTopK) &&
         E <= size_t(kMaxExperts) && quant == down_quant &&
         (quant == INFERNO_Q2_K || quant == INFERNO_Q3_K || quant == INFERNO_Q4_K);
}

int decode_chunk(size_t H) {
  if (H % 768 == 0) return 768;
  if (H % 512 == 0) return 512;
  return 256;
}

int launch_decode_layer(hipStream_t s, const DecodeArgs& a0, int quant) {
  DecodeArgs a = a0;
  a.chunk = decode_chunk(size_t(a.H));
  a.n_chunks = a.H / a.chunk;
  a.max_slots = std::min(a.E, a.T * a.k);
  const bool xsplit = a.x_dtype == INFERNO_F32;
  if ((size_t(std::max({staged_stride(a.H, xsplit), staged_stride(a.I, true),
                        a.Is ? staged_stride(a.Is, true) : 0})) +
       tile_part_floats(1) + 2 * kRows) * 4 > 160 * 1024) {
    set_error("fused decode: activation rows too long for LDS");
    return INFERNO_ERR_INVALID;
  }
  // route: grid covers E/4 x chunks workgroups (and enough threads to stage x)
  {
    const int runs = a.T * a.H / 16;
    const int gx = (a.E + 3) / 4;
    const int need = (runs + 255) / 256;
    const int gy = std::max(a.n_chunks, (need + gx - 1) / gx);
    const dim3 grid((unsigned)gx, (unsigned)gy);
    if (xsplit)
      route_kernel<float><<<grid, 256, 0, s>>>(a);
    else
      route_kernel<uint16_t><<<grid, 256, 0, s>>>(a);
    INF_LAUNCHED();
  }
  // the shared expert only needs the staged x: fork it onto the side stream
  SideStream* side = nullptr;
  int st;
  if (a.Is) {
    if ((st = side_stream(&side))) return st;
    INF_HIP(hipEventRecord(side->fork, s));
    INF_HIP(hipStreamWaitEvent(side->stream, side->fork, 0));
    if ((st = xsplit ? launch_shared<true>(side->stream, a) : launch_shared<false>(side->stream, a)))
      return st;
    INF_HIP(hipEventRecord(side->join, side->stream));
  }
  if (a.T == 1)
    select1_kernel<<<1, 64, 0, s>>>(a);
  else
    select_kernel<<<1, 1024, 0, s>>>(a);
  INF_LAUNCHED();
  switch (quant) {
    case INFERNO_Q2_K: st = xsplit ? launch_routed<INFERNO_Q2_K, true>(s, a) : launch_routed<INFERNO_Q2_K, false>(s, a); break;
    case INFERNO_Q3_K: st = xsplit ? launch_routed<INFERNO_Q3_K, true>(s, a) : launch_routed<INFERNO_Q3_K, false>(s, a); break;
    case INFERNO_Q4_K: st = xsplit ? launch_routed<INFERNO_Q4_K, true>(s, a) : launch_routed<INFERNO_Q4_K, false>(s, a); break;
    default:
      set_error("fused decode path needs Q2_K, Q3_K or Q4_K routed experts");
      return INFERNO_ERR_INVALID;
  }
  if (st) return st;
  if (a.Is) INF_HIP(hipStreamWaitEvent(s, side->join, 0));
  combine_kernel<<<unsigned((size_t(a.T) * a.H + 255) / 256), 256, 0, s>>>(a);
  INF_LAUNCHED();
  return INFERNO_OK;
}

}  // namespace inferno
