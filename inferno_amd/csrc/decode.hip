// Fused decode path of one MoE layer (T <= 64 tokens), four launches on the
// layer's stream, no events:
//
//   route    router logits as per-chunk partial sums (H split over many
//            workgroups) + staging of x into packed-f16 runs;
//   select   logits = ordered sum of the partials, exact top-k per token
//            (one wavefront each), stable dispatch (one wavefront for T = 1);
//   gate/up  routed and Q8_0 shared-expert 16-row tiles in one grid, writing
//            the SwiGLU intermediate already staged for the down pass (one
//            Q2_K bf16 token: the matrix-core kernels of decode_mfma.hpp);
//   down     8-row output tiles over all ranks plus the shared expert, with
//            out = (residual + shared) + routed summed in a fixed order,
//            deterministic without float atomics.
//
// Reference semantics: crates/model/src/laguna/gguf_model.rs:731-860 (layer
// order), gguf_moe_kernels.metal:340-565 (routed SwiGLU with the routing
// weight folded, down summed over ranks), q2_kernels.metal:2066-2235
// (shared expert plus two residual adds), moe_kernels.metal:210-238 (rank
// order combine).
#include "decode.hpp"
#include "decode_mfma.hpp"
#include "decode_runs.hpp"
#include "decode_select.hpp"

#include <cstdlib>
#include "timing.hpp"
#include "kernels.hpp"
#include "dot2_formats.hpp"
#include "routing_dev.hpp"


namespace inferno {
namespace {

constexpr int kMaxDecodeTokens = 64;

// ------------------------------------------------------------------ route

// Part `part` of the Q8_0 shared expert's gate/up tile `tile` (super-block
// columns [part * cp, part * cp + cp), cp = H / 256 / shared_parts) for the
// one token of the MFMA path, run by a workgroup of the route launch (it
// does not depend on the routing): that slice of x is staged into this
// workgroup's LDS, the packed-f16 tile kernel runs over it, and the 16
// gate and up partial sums go to shared_gu (summed in a fixed order by the
// MFMA gate/up kernel).
template <typename XT>
__device__ __forceinline__ void shared_gate_up_part(const DecodeArgs& p, int item) {
  extern __shared__ uint32_t smem[];
  constexpr bool kSplit = !std::is_same<XT, uint16_t>::value;
  const int tid = threadIdx.x, slot = (tid & 63) >> 2;
  const int H = p.H, Is = p.Is, parts = p.shared_parts;
  const int tile = item / parts, part = item % parts;
  const int Kp = H / parts, c0 = part * (Kp / kKBlock);
  const int Sx = staged_stride(Kp, kSplit);
  const size_t rb = size_t(H / kKBlock) * Fmt<INFERNO_Q8_0>::kBytes;
  const size_t off = size_t(tile * kRows + slot) * rb + size_t(c0) * Fmt<INFERNO_Q8_0>::kBytes;
  uint32_t* xs = smem;
  float* part_l = reinterpret_cast<float*>(smem + Sx);
  float* res = part_l + tile_part_floats(1, 4);
  TileDot<INFERNO_Q8_0, 2, 1, kSplit, 4, 0> td(p.sgate + off, p.sup + off, Kp);
  td.prefetch();  // quant loads in flight while x is staged
  for (int run = tid; run < Kp / 16; run += 256) {
    const XT* src = static_cast<const XT*>(p.x) + size_t(c0) * kKBlock + run * 16;
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = to_f32(src[i]);
    stage_run<kSplit>(v, xs, Kp, run);
  }
  __syncthreads();
  td.run(xs, Sx, 1, part_l, res);
  if (tid < 32) {
    const int m = tid >> 4, r = tid & 15;
    p.shared_gu[(size_t(part) * 2 + m) * Is + tile * kRows + r] = res[m * kRows + r];
  }
}

// Route launch: workgroups [0, gx * gy) compute router logit partials (and
// stage x); on the MFMA path the following Is / 16 * shared_parts
// workgroups run the shared expert's gate/up in K parts.
template <typename XT>
__global__ void __launch_bounds__(256) route_kernel(DecodeArgs p, int gx, int gy) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int T = p.T, H = p.H, E = p.E;
  const int g = blockIdx.x;
  if (g >= gx * gy) {
    shared_gate_up_part<XT>(p, g - gx * gy);
    return;
  }
  const int bx = g % gx, by = g / gx;
  // staging for the packed-f16 kernels: one thread per 16-value run of x
  if (p.stage_x) {
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
  // staging for the run gate/up kernels: a 16-lane group per 16-value run,
  // scaled for the field offsets of format xr_quant (decode_runs.hpp); fp32
  // tokens get the second (lo) f16 term
  if (p.stage_xr) {
    constexpr bool kSplit = !std::is_same<XT, uint16_t>::value;
    const int runs = H / 16, run_id = (g * 256 + tid) >> 4;
    if (run_id < T * runs) {  // uniform per 16-lane group
      const int t = run_id / runs, run = run_id % runs;
      const float v = to_f32(static_cast<const XT*>(p.x)[size_t(t) * H + run * 16 + (tid & 15)]);
      const int r16 = run & 15;
      const int shift = p.xr_quant == INFERNO_Q4_K ? runs_decode::RF<INFERNO_Q4_K>::run_shift(r16)
                                                   : runs_decode::RF<INFERNO_Q2_K>::run_shift(r16);
      runs_decode::stage_run16<kSplit>(
          v, p.stage_xr + size_t(t) * runs_decode::xrun_words(H, kSplit), H, run, shift);
    }
  }
  // staging for the MFMA gate/up: one wavefront per 256-value column
  if constexpr (std::is_same<XT, uint16_t>::value) {
    if (p.stage_xm) {
      const int cols = H / kKBlock, col_id = g * 4 + wave;
      if (col_id < T * cols) {
        const int t = col_id / cols, col = col_id % cols;
        mfma_decode::stage_column(static_cast<const uint16_t*>(p.x) + size_t(t) * H,
                                  p.stage_xm + size_t(t) * mfma_decode::stage_words(H), H, col);
      }
    }
  }
  if (p.logits_ready) return;  // uniform: the logits come from an earlier launch
  // logits partial of expert e over chunk c for every token
  const int e = bx * 4 + wave;
  const int c = by;
  if (e >= E || c >= p.n_chunks) return;
  const int h0 = c * p.chunk;
  const float* wrow = p.router + size_t(e) * H + h0;
  if (T == 1 && int(gridDim.x) == gx * gy) {
    // one token, no shared workgroups (c1: the router is the whole launch):
    // the lane's router values of the chunk (NF float4: chunks are 256, 512
    // or 768 wide) and its x values, all loads issued before the first
    // product (the loop below waits for each 256-value step's loads in
    // turn); same summation order. With shared workgroups in the launch
    // (c2, c4) they bound it, and the loop measured as fast.
    auto one = [&](auto nf_c) {
      constexpr int NF = decltype(nf_c)::value;
      float4 wv[NF];
      float xv[NF][4];
#pragma unroll
      for (int j = 0; j < NF; ++j) {
        const int i = lane * 4 + 256 * j;
        wv[j] = *reinterpret_cast<const float4*>(wrow + i);
        const XT* xr = static_cast<const XT*>(p.x) + h0 + i;
#pragma unroll
        for (int q = 0; q < 4; ++q) xv[j][q] = to_f32(xr[q]);
      }
      float a1 = 0.f;
#pragma unroll
      for (int j = 0; j < NF; ++j)
        a1 += wv[j].x * xv[j][0] + wv[j].y * xv[j][1] + wv[j].z * xv[j][2] + wv[j].w * xv[j][3];
      const float s1 = wave_sum(a1);
      if (lane == 0) p.partials[size_t(c) * E + e] = s1;
    };
    const int nf = p.chunk / 256;  // uniform; decode_chunk gives 768, 512 or 256
    if (nf == 3) one(std::integral_constant<int, 3>{});
    else if (nf == 2) one(std::integral_constant<int, 2>{});
    else one(std::integral_constant<int, 1>{});
    return;
  }
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

// Sums the chunk partials of token t into an LDS logit row with all the
// workgroup's threads; the loads of one expert's chunks are issued together.
__device__ __forceinline__ void sum_partials(const DecodeArgs& p, int t, float* logit_row,
                                             int first, int stride) {
  const int E = p.E, T = p.T;
  for (int e = first; e < E; e += stride) {
    float s = 0.f;
    for (int c0 = 0; c0 < p.n_chunks; c0 += 8) {
      float v[8];
#pragma unroll
      for (int c = 0; c < 8; ++c)
        v[c] = c0 + c < p.n_chunks  // clamped address: the eight loads go out together
                   ? p.partials[(size_t(min(c0 + c, p.n_chunks - 1)) * T + t) * E + e]
                   : 0.f;
#pragma unroll
      for (int c = 0; c < 8; ++c) s += v[c];
    }
    logit_row[e] = s;
  }
}

// The Q8_0 shared expert's down for output rows [16 g, 16 g + 16) of the one
// token (MFMA down path), run by a workgroup of the select launch: it only
// needs the shared gate/up partial sums of the route launch. Each workgroup
// forms the shared h row itself (partials summed in part order, h = silu(g)
// * u) and stages it into its LDS, so no workgroup depends on another; then
// two 8-row groups with the lane split and summation order of the shared
// part of down8_kernel. Writes ys.
constexpr int kSharedDownRows = 16;
__device__ __forceinline__ void shared_down_rows(const DecodeArgs& p, int g) {
  using FS = Fmt<INFERNO_Q8_0>;
  extern __shared__ uint32_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = (lane >> 2) & 7, sub = lane & 3, cp = lane >> 5;
  const int Is = p.Is, ubs = Is / kKBlock;
  const int Sns = staged_stride(Is, false);
  uint32_t* xss = smem;
  float* part = reinterpret_cast<float*>(xss + Sns);  // [4 wavefronts][8 rows]
  const int q_first = cp + 2 * wave;
  constexpr int kGroups = kSharedDownRows / 8;
  auto srow = [&](int grp) {
    return p.sdown + size_t(g * kSharedDownRows + grp * 8 + r) * size_t(ubs) * FS::kBytes;
  };
  // every group's first unit in flight while h is formed
  uint32_t sraw[kGroups][FS::kDw];
#pragma unroll
  for (int grp = 0; grp < kGroups; ++grp)
    if (q_first < ubs) FS::load(srow(grp) + size_t(q_first) * FS::kBytes, sub, sraw[grp]);
  form_shared_h<256>(p, xss, tid);
  __syncthreads();
#pragma unroll
  for (int grp = 0; grp < kGroups; ++grp) {
    float accs = 0.f;
    for (int q = q_first; q < ubs; q += 8) {
      if (q != q_first) FS::load(srow(grp) + size_t(q) * FS::kBytes, sub, sraw[grp]);
      accs += FS::dot(sraw[grp], sub, xrow_at<false>(xss, Is, q));
    }
    accs += __shfl_xor(accs, 1, kWave);
    accs += __shfl_xor(accs, 2, kWave);
    accs += __shfl_xor(accs, 32, kWave);
    if ((lane & 35) == 0) part[wave * 8 + r] = accs;
    __syncthreads();
    if (tid < 8)
      p.ys[size_t(g) * kSharedDownRows + grp * 8 + tid] =
          ((part[tid] + part[8 + tid]) + part[16 + tid]) + part[24 + tid];
    __syncthreads();
  }
}

// Workgroup 0 sums the partials and selects; on the MFMA down path
// workgroups 1.. run the shared expert's down (shared_down_rows).
__global__ void __launch_bounds__(256) select1_kernel(DecodeArgs p) {
  if (blockIdx.x > 0) {
    shared_down_rows(p, int(blockIdx.x) - 1);
    return;
  }
  __shared__ float logit_row[kMaxExperts];
  __shared__ float bias[kMaxExperts];
  __shared__ Top1Lds tk;
  // the selection is a serial chain: its waves go first on SIMDs shared with
  // shared-down workgroups
  __builtin_amdgcn_s_setprio(3);
  const int tid = threadIdx.x;
  const int E = p.E;
  // the bias load is issued before the partials' loads and stored after
  // them, so the two round trips overlap (E <= 256: one expert per thread)
  const float bv = (p.bias && tid < E) ? p.bias[tid] : 0.f;
  sum_partials(p, 0, logit_row, tid, 256);
  bias[tid] = bv;
  __syncthreads();
  if (tid >= 64) return;
  float lg[4], bs[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = tid + 64 * j;
    lg[j] = e < E ? logit_row[e] : 0.f;
    bs[j] = bias[e];
  }
  topk1_wave(lg, bs, E, p.k, p.score_fn, p.norm, p.scale, &tk);
  select1_write(p, &tk);
}

__global__ void __launch_bounds__(1024) select_kernel(DecodeArgs p) {
  __shared__ float logit_row[16][kMaxExperts];
  __shared__ float bias[kMaxExperts];
  __shared__ uint32_t ids_lds[kMaxDecodeTokens * kMaxTopK];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int T = p.T, E = p.E, k = p.k;
  if (p.bias)
    for (int e = tid; e < E; e += 1024) bias[e] = p.bias[e];
  __syncthreads();
  for (int t = wave; t < T; t += 16) {
    sum_partials(p, t, logit_row[wave], lane, 64);
    __builtin_amdgcn_wave_barrier();  // LDS is in order within a wavefront
    uint32_t sel[kMaxTopK];
    topk_row_wave(logit_row[wave], p.bias ? bias : nullptr, E, k, p.score_fn, p.norm, p.scale, t,
                  p.ids, p.weights, nullptr, sel);
#pragma unroll
    for (int r = 0; r < kMaxTopK; ++r)
      if (r < k && lane == r) ids_lds[t * k + r] = sel[r];
  }
  __syncthreads();
  dispatch_block(ids_lds, T * k, E, p.offsets, p.sorted, p.active);
  // per-slot work descriptors; dispatch_block ended with a barrier, which
  // orders this workgroup's global writes before these reads
  const uint32_t n = p.active[0];
  for (uint32_t j = tid; j < n; j += 1024) {
    const uint32_t e = p.active[1 + j], lo = p.offsets[e];
    p.slots[j] = make_uint4(e, lo, p.offsets[e + 1], p.sorted[lo]);
  }
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

// Waves per SIMD the decode kernels are compiled for: two when a wavefront
// holds four or more columns' quant bytes at once (256 registers), else three.
template <int KU>
struct DecodeOcc {
  static constexpr int value = KU >= 2 ? 2 : 3;
};

// Largest column batch per wavefront that fits 256 registers without
// spilling, by format and activation layout (gate/up holds two matrices).
template <int Q, bool SPLIT>
struct GateUpMaxKU {
  static constexpr int value = Q == INFERNO_Q2_K ? (SPLIT ? 4 : 6)
                               : Q == INFERNO_Q4_K ? (SPLIT ? 2 : 4)
                                                   : (SPLIT ? 1 : 2);
};

// One 16-row gate/up tile: routed (tile `item` of the active slots) or the
// Q8_0 shared expert (tile `item` of its rows).
template <int Q, bool XSPLIT, bool SHARED, int WAVES, int KU>
__device__ __forceinline__ void gate_up_tile(const DecodeArgs& p, uint32_t item) {
  extern __shared__ uint32_t smem[];
  const int tid = threadIdx.x, slot = (tid & 63) >> 2;
  const int T = p.T, H = p.H, I = p.I, Is = p.Is, k = p.k;
  const int Sx = staged_stride(H, XSPLIT);
  const int tiles_i = I / kRows;
  constexpr bool shared = SHARED;
  uint32_t lo = 0, hi = uint32_t(T), first = 0;
  int tile = int(item);
  const uint8_t *r0, *r1;
  const size_t rb = size_t(H / kKBlock) * Fmt<Q>::kBytes;
  if constexpr (!shared) {
    const uint32_t j = item / uint32_t(tiles_i);
    const uint4 sl = p.slots[j];  // read before the bound check: one round trip
    if (j >= p.active[0]) return;
    tile = int(item % uint32_t(tiles_i));
    const size_t off = size_t(sl.x) * p.gate_stride + size_t(tile * kRows + slot) * rb;
    r0 = p.gate + off;
    r1 = p.up + off;
    lo = sl.y;
    hi = sl.z;
    first = sl.w;
  } else {
    r0 = p.sgate + size_t(tile * kRows + slot) * rb;
    r1 = p.sup + size_t(tile * kRows + slot) * rb;
  }
  uint32_t* xs = smem;
  float* part = reinterpret_cast<float*>(smem + Sx);
  float* res = part + tile_part_floats(1, WAVES);
  TileDot<Q, 2, 1, XSPLIT, WAVES, KU> td(r0, r1, H);
  for (uint32_t c = lo; c < hi; ++c) {
    const uint32_t a = shared ? c : (c == lo ? first : p.sorted[c]);
    const uint32_t tok = shared ? c : a / uint32_t(k);
    td.prefetch();  // quant loads in flight while x is copied
    copy_rows_to_lds<64 * WAVES>(xs, Sx, 1, [&](int) { return p.stage_x + size_t(tok) * Sx; });
    __syncthreads();
    td.run(xs, Sx, 1, part, res);
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

// gate/up launch: the shared expert's tiles and the routed tiles in one grid.
template <int Q, bool XSPLIT, int KU>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DecodeOcc<KU>::value, 8)))
    gate_up_kernel(DecodeArgs p) {
  // the shared expert's tiles (3.2x the bytes of a routed Q2_K tile) are
  // dispatched first, so that the routed tiles fill in behind them instead
  // of the big tiles forming a tail on part of the chip
  const uint32_t item = blockIdx.x;
  const uint32_t nshared = uint32_t(p.Is / kRows);
  if (item < nshared)
    gate_up_tile<INFERNO_Q8_0, XSPLIT, true, 4, 0>(p, item);
  else
    gate_up_tile<Q, XSPLIT, false, 4, KU>(p, item - nshared);
}

// Routed down with the combine folded in, 8-row output tiles: workgroup =
// (token t, 8 output rows), which makes T * H / 8 workgroups (768 for a
// 6144-wide token: three per CU, one round). Lane = (column parity cp, row
// r, sub); a lane group (wavefront, cp) takes the (rank, super-block column)
// pairs q = cp + 2 wave + 8 u, with all KU of them in flight at once. The
// token's k SwiGLU rows are copied to LDS as their f16 high parts only
// (plus run sums and scales): about 2^-12 relative rounding per element.
// Lane groups meet in registers (cp) and LDS (wavefronts) in a fixed order;
// out = (residual + shared) + routed, deterministic without float atomics.
template <int Q, int KU>
__global__ void __launch_bounds__(256)
    __attribute__((amdgpu_waves_per_eu(Q == INFERNO_Q2_K ? 3 : 2, 8))) down8_kernel(DecodeArgs p) {
  using F = Fmt<Q>;
  extern __shared__ uint32_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = (lane >> 2) & 7, sub = lane & 3, cp = lane >> 5;
  const int H = p.H, I = p.I, k = p.k;
  const int tiles_h = H / 8;
  const int t = int(blockIdx.x) / tiles_h, tile = int(blockIdx.x) % tiles_h;
  const int Ss = staged_stride(I, true), Sn = staged_stride(I, false);
  const int Sns = p.Is ? staged_stride(p.Is, false) : 0;
  uint32_t* xs = smem;                  // k routed rows + the shared row, non-split layout
  uint32_t* xss = smem + k * Sn;
  float* part = reinterpret_cast<float*>(xss + Sns);  // [2][4 wavefronts][8 rows]
  const int bpr = I / kKBlock;
  const size_t rb = size_t(bpr) * F::kBytes;
  const uint8_t* wrow = p.down + size_t(tile * 8 + r) * rb;
  const uint32_t* ids = p.ids + size_t(t) * k;
  const int nq = k * bpr;
  uint32_t raw[KU][F::kDw];
  auto issue = [&](int q0) {
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int q = q0 + 8 * u;
      if (q < nq) {
        const int rank = q / bpr, col = q - rank * bpr;
        F::load(wrow + size_t(ids[rank]) * p.down_stride + size_t(col) * F::kBytes, sub, raw[u]);
      }
    }
  };
  const int q_first = cp + 2 * wave;
  issue(q_first);  // quant loads in flight while the h rows are copied
  // the shared expert: 8 rows of its down matrix against the token's shared
  // h row, one Q8_0 unit (256 values) per lane group and step
  using FS = Fmt<INFERNO_Q8_0>;
  const int Is = p.Is, ubs = Is / kKBlock;
  const uint8_t* srow =
      Is ? p.sdown + size_t(tile * 8 + r) * size_t(ubs) * FS::kBytes : nullptr;
  uint32_t sraw[FS::kDw];
  if (Is && q_first < ubs) FS::load(srow + size_t(q_first) * FS::kBytes, sub, sraw);
  // staged h rows t*k .. t*k+k-1: copy the high pairs and the run sums/scales
  {
    const int hi4 = I / 8, tail4 = I / 32;  // uint4 words of the two parts
    const int per = hi4 + tail4;
    for (int i = tid; i < k * per; i += 256) {
      const int rank = i / per, w = i - rank * per;
      const uint4* from = reinterpret_cast<const uint4*>(p.stage_h + size_t(t * k + rank) * Ss);
      uint4* to = reinterpret_cast<uint4*>(xs + rank * Sn);
      // the high pairs are the first I/2 words, the sums/scales the last I/8
      to[w] = w < hi4 ? from[w] : from[w + hi4];
    }
    if (Is) {
      const int shi4 = Is / 8, sper = shi4 + Is / 32;
      const uint4* from =
          reinterpret_cast<const uint4*>(p.stage_hs + size_t(t) * staged_stride(Is, true));
      uint4* to = reinterpret_cast<uint4*>(xss);
      for (int w = tid; w < sper; w += 256) to[w] = w < shi4 ? from[w] : from[w + shi4];
    }
  }
  __syncthreads();
  float acc = 0.f;
  for (int q0 = q_first; q0 < nq; q0 += 8 * KU) {
    if (q0 != q_first) issue(q0);
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int q = q0 + 8 * u;
      if (q < nq) {
        const int rank = q / bpr, col = q - rank * bpr;
        acc += F::dot(raw[u], sub, xrow_at<false>(xs + rank * Sn, I, col));
      }
    }
  }
  float accs = 0.f;
  for (int q = q_first; q < ubs; q += 8) {
    if (q != q_first) FS::load(srow + size_t(q) * FS::kBytes, sub, sraw);
    accs += FS::dot(sraw, sub, xrow_at<false>(xss, Is, q));
  }
  acc += __shfl_xor(acc, 1, kWave);
  acc += __shfl_xor(acc, 2, kWave);
  acc += __shfl_xor(acc, 32, kWave);
  accs += __shfl_xor(accs, 1, kWave);
  accs += __shfl_xor(accs, 2, kWave);
  accs += __shfl_xor(accs, 32, kWave);
  if ((lane & 35) == 0) {  // sub == 0, cp == 0
    part[wave * 8 + r] = acc;
    part[32 + wave * 8 + r] = accs;
  }
  __syncthreads();
  if (tid < 8) {
    const float v = ((part[tid] + part[8 + tid]) + part[16 + tid]) + part[24 + tid];
    const float vs = ((part[32 + tid] + part[40 + tid]) + part[48 + tid]) + part[56 + tid];
    const size_t o = size_t(t) * H + size_t(tile) * 8 + tid;
    p.out[o] = ((p.residual ? p.residual[o] : 0.f) + vs) + v;
  }
}

// Routed gate/up: four wavefronts per 16-row tile, each with its quant loads
// for KU columns in flight at once.
size_t gate_up_lds(int H, bool xsplit) {
  return (size_t(staged_stride(H, xsplit)) + tile_part_floats(1) + 2 * kRows) * 4;
}

template <int Q, bool XSPLIT, int KU>
void launch_gate_up_ku(hipStream_t s, const DecodeArgs& a) {
  const size_t tiles = size_t(a.routed_tiles) + (a.Is ? size_t(a.Is / kRows) : 0);
  gate_up_kernel<Q, XSPLIT, KU><<<unsigned(tiles), 256, gate_up_lds(a.H, XSPLIT), s>>>(a);
}

// columns per wavefront: ceil(H / 256 / 4), capped by the format (a longer
// row loops over batches)
template <int Q, bool XSPLIT>
void launch_gate_up(hipStream_t s, const DecodeArgs& a) {
  constexpr int kMax = GateUpMaxKU<Q, XSPLIT>::value;
  const int per = (a.H / kKBlock + 3) / 4;
  if (per <= 1 || kMax == 1) launch_gate_up_ku<Q, XSPLIT, 1>(s, a);
  else if (per <= 2 || kMax == 2) launch_gate_up_ku<Q, XSPLIT, (kMax < 2 ? kMax : 2)>(s, a);
  else if (per <= 4 || kMax == 4) launch_gate_up_ku<Q, XSPLIT, (kMax < 4 ? kMax : 4)>(s, a);
  else launch_gate_up_ku<Q, XSPLIT, kMax>(s, a);
}

size_t down8_lds(int k, int I, int Is) {
  return (size_t(k) * staged_stride(I, false) + (Is ? size_t(staged_stride(Is, false)) : 0) +
          2 * 4 * 8) * 4;
}

template <int Q>
void launch_down(hipStream_t s, const DecodeArgs& a) {
  const unsigned grid = unsigned(size_t(a.T) * (a.H / 8));
  const size_t lds = down8_lds(a.k, a.I, a.Is);
  const int per = (a.k * (a.I / kKBlock) + 7) / 8;
  // Q3_K holds four pairs per batch without spilling, the others eight
  constexpr int kMax8 = Q == INFERNO_Q3_K ? 4 : 8;
  if (per <= 4 || kMax8 == 4)
    down8_kernel<Q, 4><<<grid, 256, lds, s>>>(a);
  else
    down8_kernel<Q, kMax8><<<grid, 256, lds, s>>>(a);
}

int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cus[dev] && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus[dev] = 0;
  return cus[dev];
}

// Routed Q2_K gate/up for one bf16 token on the matrix cores
// (decode_mfma.hpp); on by default, INFERNO_DECODE_MFMA=0 turns it off.
bool mfma_enabled() {
  return !switch_off("INFERNO_DECODE_MFMA");
}

// K parts of the shared gate/up on the MFMA path: the fewest parts (each
// re-read of the partial sums costs the gate/up prologue) that divide the
// super-block columns and give the route launch at least two shared
// workgroups per CU (16-row tiles x parts), else the most that divide them,
// at most kMaxSharedParts. c2 (Is 2048, 24 columns): 4; c4 (Is 1536, 16
// columns): 8, measured 2.8 us per 4-layer step faster than 4. The part
// count sets the order in which the shared partial sums are added, so it
// depends on the shape only, never on the device: the CU count is MI355X's
// (256) whatever the device reports, and the same layer gives the same bits
// on any device.
constexpr int kPartsCUs = 256;
int shared_parts(int H, int Is) {
  const int cols = H / kKBlock, tiles = Is / kRows, want = 2 * kPartsCUs;
  int best = 1;
  for (int k = 2; k <= kMaxSharedParts; ++k) {
    if (cols % k) continue;
    best = k;
    if (tiles * k >= want) return k;
  }
  return best;
}

// The fp8 x fp4 gate/up: one bf16 token, Q2_K (NB a multiple of 4, 4..28)
// or Q3_K (NB a multiple of 8, 8..24).
bool mfma_gate_up_covers(const DecodeArgs& a, int quant) {
  const int NB = a.H / kKBlock;
  const bool shape = quant == INFERNO_Q2_K ? mfma_decode::covers_width(a.H)
                     : quant == INFERNO_Q3_K ? (a.H % kKBlock == 0 && NB % 8 == 0 && NB >= 8 && NB <= 24)
                                             : false;
  return mfma_enabled() && a.T == 1 && shape && a.x_dtype == INFERNO_BF16 &&
         (a.Is == 0 || a.shared_gu != nullptr) && a.I % kRows == 0 &&
         mfma_decode::lds_bytes(a.H, quant) <= 160 * 1024 && a.stage_xm != nullptr &&
         device_cus() > 0;
}

template <int Q, int NB, int SP>
int launch_gate_up_mfma_sp(hipStream_t s, const DecodeArgs& a, int ntiles) {
  constexpr bool SEL = SP > 0;
  static bool attr = false;
  auto* kern = mfma_decode::gate_up_fp4_kernel<Q, NB, SEL, SEL ? SP : 4>;
  if (!attr) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024) != hipSuccess) {
      set_error("MFMA gate/up kernel: cannot raise its LDS limit");
      return INFERNO_ERR_DEVICE;
    }
    attr = true;
  }
  const unsigned grid = unsigned(std::min(ntiles, device_cus()));
  kern<<<grid, mfma_decode::kThreads, mfma_decode::lds_bytes(a.H, Q, SEL, (a.Is && a.ys) ? a.Is : 0), s>>>(a, ntiles);
  INF_LAUNCHED();
  return INFERNO_OK;
}

template <int Q, int NB, bool SEL>
int launch_gate_up_mfma_nb(hipStream_t s, const DecodeArgs& a, int ntiles) {
  // H = 4096 (the Laguna-S width) also has an instance whose selection
  // takes routers of at most 128 experts with two slots per lane
  if constexpr (SEL && NB == 16) {
    if (a.E <= 2 * kWave) return launch_gate_up_mfma_sp<Q, NB, 2>(s, a, ntiles);
  }
  return launch_gate_up_mfma_sp<Q, NB, SEL ? 4 : 0>(s, a, ntiles);
}

template <int Q, bool SEL>
int launch_gate_up_mfma_q(hipStream_t s, const DecodeArgs& a0, int ntiles) {
  if constexpr (Q == INFERNO_Q3_K) {
    switch (a0.H / kKBlock) {
      case 8: return launch_gate_up_mfma_nb<Q, 8, SEL>(s, a0, ntiles);
      case 16: return launch_gate_up_mfma_nb<Q, 16, SEL>(s, a0, ntiles);
      default: return launch_gate_up_mfma_nb<Q, 24, SEL>(s, a0, ntiles);
    }
  } else {
    switch (a0.H / kKBlock) {
      case 4: return launch_gate_up_mfma_nb<Q, 4, SEL>(s, a0, ntiles);
      case 8: return launch_gate_up_mfma_nb<Q, 8, SEL>(s, a0, ntiles);
      case 12: return launch_gate_up_mfma_nb<Q, 12, SEL>(s, a0, ntiles);
      case 16: return launch_gate_up_mfma_nb<Q, 16, SEL>(s, a0, ntiles);
      case 20: return launch_gate_up_mfma_nb<Q, 20, SEL>(s, a0, ntiles);
      case 24: return launch_gate_up_mfma_nb<Q, 24, SEL>(s, a0, ntiles);
      default: return launch_gate_up_mfma_nb<Q, 28, SEL>(s, a0, ntiles);
    }
  }
}

// The routed tiles of the k slots on the fp8 x fp4 kernel (the shared
// expert's gate/up already ran in the route launch); with sel, the kernel
// also selects and runs the shared down (no select launch).
int launch_gate_up_mfma(hipStream_t s, const DecodeArgs& a0, int quant, bool sel) {
  const int ntiles = a0.max_slots * (a0.I / kRows);
  if (quant == INFERNO_Q3_K)
    return sel ? launch_gate_up_mfma_q<INFERNO_Q3_K, true>(s, a0, ntiles)
               : launch_gate_up_mfma_q<INFERNO_Q3_K, false>(s, a0, ntiles);
  return sel ? launch_gate_up_mfma_q<INFERNO_Q2_K, true>(s, a0, ntiles)
             : launch_gate_up_mfma_q<INFERNO_Q2_K, false>(s, a0, ntiles);
}

// The selection (and the shared down) in the fp8 x fp4 gate/up launch: one
// token, at most three shared-down octets per workgroup (kSdWpo wavefronts
// each, one 256-value unit per lane, each wavefront's rows copied to its own
// LDS area during the selection); INFERNO_DECODE_SEL=0 keeps the select launch.
bool sel_in_gate_up(const DecodeArgs& a, bool shared_down_here) {
  if (a.T != 1 || switch_off("INFERNO_DECODE_SEL")) return false;
  const int ntiles = a.max_slots * (a.I / kRows);
  const int grid = std::min(ntiles, device_cus());
  if (!shared_down_here) return mfma_decode::lds_bytes(a.H, a.xr_quant, true, 0) <= 160 * 1024;
  const int rw = 8 * ((a.H / 8 + grid - 1) / grid);  // the workgroup's rows, whole octets
  return a.Is % kKBlock == 0 && a.Is <= 2 * kKBlock * kSdWpo && a.H % 8 == 0 &&
         rw <= 8 * kSdMaxOctets && mfma_decode::lds_bytes(a.H, a.xr_quant, true, a.Is) <= 160 * 1024;
}

template <int TR, int PER>
int launch_down_mfma_per(hipStream_t s, const DecodeArgs& a) {
  static bool attr = false;
  auto* kern = mfma_decode::down_q2k_kernel<8, TR, PER>;
  if (!attr) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024) != hipSuccess) {
      set_error("MFMA down kernel: cannot raise its LDS limit");
      return INFERNO_ERR_DEVICE;
    }
    attr = true;
  }
  const int ntiles = a.H / TR;
  const unsigned grid = unsigned(std::min(ntiles, device_cus()));
  kern<<<grid, mfma_decode::kThreads, mfma_decode::down_lds_bytes(a.I), s>>>(a, ntiles);
  INF_LAUNCHED();
  return INFERNO_OK;
}

template <int TR>
int launch_down_mfma_tr(hipStream_t s, const DecodeArgs& a) {
  switch (mfma_decode::down_chunks_per_thread(8, a.k, TR)) {
    case 1: return launch_down_mfma_per<TR, 1>(s, a);
    case 2: return launch_down_mfma_per<TR, 2>(s, a);
    case 3: return launch_down_mfma_per<TR, 3>(s, a);
    case 4: return launch_down_mfma_per<TR, 4>(s, a);
    case 5: return launch_down_mfma_per<TR, 5>(s, a);
    default: return launch_down_mfma_per<TR, 6>(s, a);
  }
}

// Routed down for one token on the MFMA kernel (I = 2048: 8 super-block
// columns; k <= 8 ranks). 12-row tiles when they split H into a whole
// number of rounds of one tile per CU, else 16-row tiles.
// Rows per tile of the Q2_K MFMA down for a layer of width H.
int down_tile_rows(int H) {
  const int cus = device_cus();
  return (H % 12 == 0 && (H / 12) % cus == 0 && (H / 16) % cus != 0) ? 12 : 16;
}

int launch_down_mfma(hipStream_t s, const DecodeArgs& a) {
  if (down_tile_rows(a.H) == 12) return launch_down_mfma_tr<12>(s, a);
  return launch_down_mfma_tr<16>(s, a);
}

// Route launch: router logit partials over E/4 x chunks workgroups (none
// when the logits are ready), enough of them to stage x for the expert
// kernels, then shared_wgs workgroups of the shared gate/up in K parts.
int launch_route(hipStream_t s, const DecodeArgs& a, int shared_wgs) {
  const bool xsplit = a.x_dtype == INFERNO_F32;
  const int runs = a.T * a.H / 16;
  const int need = std::max(std::max((runs + 255) / 256, (a.T * (a.H / kKBlock) + 3) / 4),
                            a.stage_xr ? (a.T * a.H + 255) / 256 : 0);
  const int gx = a.logits_ready ? 1 : (a.E + 3) / 4;
  const int gy = a.logits_ready ? need : std::max(a.n_chunks, (need + gx - 1) / gx);
  const unsigned grid = unsigned(gx * gy + shared_wgs);
  const size_t lds = shared_wgs ? gate_up_lds(a.H / a.shared_parts, xsplit) : 0;
  return timed(s, kTimerRoute,
               shared_wgs ? "route+shared: route_kernel (router logit partials, Q8_0 "
                            "shared gate/up in K parts)"
                          : "route: route_kernel (router logit partials, x staging)",
               [&] {
                 if (xsplit)
                   route_kernel<float><<<grid, 256, lds, s>>>(a, gx, gy);
                 else
                   route_kernel<uint16_t><<<grid, 256, lds, s>>>(a, gx, gy);
                 INF_LAUNCHED();
                 return INFERNO_OK;
               });
}

// One token whose shared expert has the routed formats and width (the
// Laguna XS layer, crates/backend/src/metal/laguna_xs.rs:1001-1144: the
// shared expert as a ninth assignment of weight 1 next to the eight routed
// ones): three launches, route (logits, x as f16 runs), the selecting run
// gate/up over k + 1 slots, the run down summing k + 1 ranks plus the
// residual.
int launch_decode_shared_slot(hipStream_t s, DecodeArgs a, int quant) {
  a.stage_x = nullptr;
  a.stage_xm = nullptr;
  a.xr_quant = quant;
  a.h_mfma = 1;
  a.ys = nullptr;
  // the down launch's first tiles (k + 1 ranks), warmed in L2 by the
  // selecting gate/up launch under its last tile (INFERNO_DECODE_WARM_DOWN=0: off)
  a.dpf_rows = a.dpf_row_bytes = 0;
  if (!switch_off("INFERNO_DECODE_WARM_DOWN")) {
    a.dpf_rows = runs_down_tile_rows(a.h_quant, a.H, a.I, a.k + 1);
    a.dpf_row_bytes = runs_down_row_bytes(a.h_quant, a.I);
  }
  a.max_slots = a.k;
  if (int st = launch_route(s, a, 0)) return st;
  int st = timed(s, kTimerGateUp,
                 "runs+shared+select: gate_up_runs_multi_kernel (top-k in every workgroup's "
                 "prologue; the routed tiles and the shared expert's as assignment k on f16 MFMA)",
                 [&] { return launch_gate_up_runs_multi(s, a, quant, true); });
  if (st) return st;
  return timed(s, kTimerDown,
               "runs-down+shared: down_runs_kernel (routed and shared down on f16 MFMA + "
               "residual)",
               [&] { return launch_down_runs(s, a, a.h_quant); });
}

}  // namespace

bool decode_shared_slot_supported(size_t T, size_t k, size_t E, size_t H, size_t I, int x_dtype,
                                  int quant, int down_quant) {
  return T == 1 && k >= 1 && k <= size_t(kMaxTopK) && E <= size_t(kMaxExperts) &&
         H % kKBlock == 0 && I % kKBlock == 0 && mfma_enabled() &&
         !switch_off("INFERNO_DECODE_SHARED_SLOT") &&
         (quant == INFERNO_Q2_K || quant == INFERNO_Q3_K || quant == INFERNO_Q4_K) &&
         runs_multi_sel_covers(quant, int(H), x_dtype) &&
         runs_down_covers(down_quant, int(H), int(I), int(k) + 1);
}

size_t decode_mfma_stage_words(size_t H) { return size_t(mfma_decode::stage_words(int(H))); }
size_t decode_shared_partial_floats(size_t H, size_t Is) {
  (void)H;  // room for the most parts any shape takes
  return size_t(kMaxSharedParts) * 2 * Is;
}

bool decode_supported(size_t T, size_t k, size_t E, size_t H, size_t I, size_t Is, int x_dtype,
                      int quant, int down_quant) {
  if (!(T >= 1 && T <= size_t(kMaxDecodeTokens) && E <= size_t(kMaxExperts) && k <= size_t(kMaxTopK) &&
        quant == down_quant &&
        (quant == INFERNO_Q2_K || quant == INFERNO_Q3_K || quant == INFERNO_Q4_K)))
    return false;
  const size_t kLds = 160 * 1024;
  return gate_up_lds(int(H), x_dtype == INFERNO_F32) <= kLds &&
         down8_lds(int(k), int(I), int(Is)) <= kLds;
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
  if (a.logits_ready) {  // one "chunk": the logits themselves
    a.partials = const_cast<float*>(a.logits_ready);
    a.chunk = a.H;
    a.n_chunks = 1;
  }
  a.max_slots = std::min(a.E, a.T * a.k);
  if (a.shared_slot) return launch_decode_shared_slot(s, a, quant);
  a.h_quant = quant;
  const bool xsplit = a.x_dtype == INFERNO_F32;
  // gate/up: fp8 x fp4 matrix-core kernel (one Q2_K bf16 token), else the
  // f16-run matrix-core kernel (one token, any routed format, with its down
  // kernel), else the packed-f16 tile kernels
  const bool shared_down_ok = a.H % kSharedDownRows == 0 && a.Is % kKBlock == 0 &&
                              (a.Is == 0 || a.ys != nullptr);
  const bool use_fp4 = mfma_gate_up_covers(a, quant);
  // (bf16 tokens here; one fp32 token takes the grouped run gate/up below)
  const bool use_runs = !use_fp4 && mfma_enabled() && a.T == 1 && a.x_dtype == INFERNO_BF16 &&
                        shared_down_ok &&
                        (a.Is == 0 || a.shared_gu != nullptr) && a.stage_xr != nullptr &&
                        a.I % kRows == 0 && runs_gate_up_covers(quant, a.H, a.x_dtype) &&
                        runs_down_covers(quant, a.H, a.I, a.k);
  // one fp32 token: the grouped run gate/up (two f16 terms per run; it takes
  // the one-token slots as they are) with the one-token run down
  const bool use_runs32 = !use_fp4 && mfma_enabled() && !switch_off("INFERNO_DECODE_RUNS_F32") &&
                          a.T == 1 && a.x_dtype == INFERNO_F32 && shared_down_ok &&
                          (a.Is == 0 || a.shared_gu != nullptr) && a.stage_xr != nullptr &&
                          a.I % kRows == 0 && runs_multi_covers(quant, a.H, a.I, a.x_dtype) &&
                          runs_down_covers(quant, a.H, a.I, a.k);
  // several tokens, no shared expert: the run kernels grouped by expert
  const bool use_multi = !use_fp4 && !use_runs && mfma_enabled() && a.T > 1 && a.Is == 0 &&
                         a.y != nullptr && a.stage_xr != nullptr && a.I % kRows == 0 &&
                         runs_multi_covers(quant, a.H, a.I, a.x_dtype);
  const bool use_mfma = use_fp4 || use_runs || use_runs32;
  // with a matrix-core gate/up the shared expert's gate/up runs in the route
  // launch and stages its own x; otherwise x is staged for the tile kernels
  a.shared_parts = shared_parts(a.H, a.Is);
  if (use_mfma || use_multi) a.stage_x = nullptr;
  if (!use_fp4) a.stage_xm = nullptr;
  if (!use_runs && !use_runs32 && !use_multi) a.stage_xr = nullptr;
  a.xr_quant = quant;
  // down after a matrix-core gate/up (h in the run layout): the Q2_K kernel
  // (I = 2048, k <= 8) or the run kernel; the shared down then runs in the
  // select launch
  const bool use_q2k_down = use_fp4 && quant == INFERNO_Q2_K && mfma_decode::down_covers(a.I, a.k) &&
                            shared_down_ok &&
                            mfma_decode::down_lds_bytes(a.I) <= 160 * 1024;
  const bool use_runs_down = !use_q2k_down && use_mfma && shared_down_ok &&
                             runs_down_covers(quant, a.H, a.I, a.k);
  const bool use_mfma_down = use_q2k_down || use_runs_down;
  a.h_mfma = (use_mfma_down || use_multi) ? 1 : 0;
  // the down launch's first tiles, warmed in L2 by the selecting gate/up
  // launch under its last routed tile (INFERNO_DECODE_WARM_DOWN=0: off)
  a.dpf_rows = a.dpf_row_bytes = 0;
  if (a.T == 1 && !switch_off("INFERNO_DECODE_WARM_DOWN")) {
    if (use_q2k_down) {
      a.dpf_rows = down_tile_rows(a.H);
      a.dpf_row_bytes = a.I / kKBlock * mfma_decode::kQ2Bytes;
    } else if (use_runs_down) {
      a.dpf_rows = runs_down_tile_rows(quant, a.H, a.I, a.k);
      a.dpf_row_bytes = runs_down_row_bytes(quant, a.I);
    }
  }
  // the shared down output ys exists only with a shared expert on that path
  if (!use_mfma_down || a.Is == 0) a.ys = nullptr;
  if (!decode_supported(a.T, a.k, a.E, a.H, a.I, a.Is, a.x_dtype, quant, quant)) {
    set_error("fused decode path does not cover this layer shape");
    return INFERNO_ERR_INVALID;
  }
  {
    const int shared_wgs = use_mfma ? a.Is / kRows * a.shared_parts : 0;
    if (int st = launch_route(s, a, shared_wgs)) return st;
  }
  // one token on the fp8 x fp4 gate/up: the selection and the shared down
  // run in the gate/up launch (no select launch)
  // one fp32 token on the grouped run gate/up without a shared expert: the
  // selection moves into that launch too
  const bool use_sel32 = use_runs32 && a.T == 1 && a.Is == 0 && !switch_off("INFERNO_DECODE_SEL") &&
                         runs_multi_sel_covers(quant, a.H, a.x_dtype);
  const bool use_sel = use_sel32 || (use_fp4 && sel_in_gate_up(a, use_mfma_down && a.Is));
  if (!use_sel) {
    const int sd_wgs = (use_mfma_down && a.Is) ? a.H / kSharedDownRows : 0;
    const size_t sd_lds = sd_wgs ? (size_t(staged_stride(a.Is, false)) + 32) * 4 : 0;
    const char* label = a.T != 1 ? "select: select_kernel"
                        : sd_wgs ? "select+shared-down: select1_kernel (top-k, dispatch; Q8_0 shared down)"
                                 : "select: select1_kernel";
    const int st = timed(s, kTimerSelect, label, [&] {
      if (a.T == 1)
        select1_kernel<<<1 + sd_wgs, 256, sd_lds, s>>>(a);
      else
        select_kernel<<<1, 1024, 0, s>>>(a);
      INF_LAUNCHED();
      return INFERNO_OK;
    });
    if (st) return st;
  }
  // gate/up (routed tiles, plus the shared tiles when they did not run in
  // the route launch), then the routed down with the shared down and the
  // residual folded in: one stream, no events
  a.routed_tiles = a.max_slots * (a.I / kRows);
  const char* gu_label =
      (use_sel && use_fp4) ? "mfma+select: gate_up_fp4_kernel (top-k and Q8_0 shared down in every workgroup's prologue; routed tiles on fp8 x fp4 MFMA; shared gate/up in the route launch)"
      : use_fp4 ? "mfma: gate_up_fp4_kernel (routed tiles on fp8 x fp4 MFMA; shared gate/up in the route launch)"
      : use_runs ? "runs: gate_up_runs_kernel (routed tiles on f16 MFMA; shared gate/up in the route launch)"
      : use_sel32 ? "runs32+select: gate_up_runs_multi_kernel (top-k in every workgroup's prologue; routed tiles on f16 MFMA, fp32 token as two f16 terms)"
      : use_runs32 ? "runs32: gate_up_runs_multi_kernel (routed tiles on f16 MFMA, fp32 token as two f16 terms; shared gate/up in the route launch)"
      : use_multi ? "runs-multi: gate_up_runs_multi_kernel (each expert's routed tiles for all its tokens on f16 MFMA)"
                  : "tiles: gate_up_kernel (routed + Q8_0 shared tiles)";
  int st = timed(s, kTimerGateUp, gu_label, [&]() -> int {
    if (use_fp4) return launch_gate_up_mfma(s, a, quant, use_sel);
    if (use_runs) return launch_gate_up_runs(s, a, quant);
    if (use_multi || use_runs32) return launch_gate_up_runs_multi(s, a, quant, use_sel32);
    switch (quant) {
      case INFERNO_Q2_K: xsplit ? launch_gate_up<INFERNO_Q2_K, true>(s, a) : launch_gate_up<INFERNO_Q2_K, false>(s, a); break;
      case INFERNO_Q3_K: xsplit ? launch_gate_up<INFERNO_Q3_K, true>(s, a) : launch_gate_up<INFERNO_Q3_K, false>(s, a); break;
      default: xsplit ? launch_gate_up<INFERNO_Q4_K, true>(s, a) : launch_gate_up<INFERNO_Q4_K, false>(s, a); break;
    }
    INF_LAUNCHED();
    return INFERNO_OK;
  });
  if (st) return st;
  if (use_q2k_down)
    return timed(s, kTimerDown,
                 "mfma-down: down_q2k_kernel (routed Q2_K down on MFMA + combine; shared down "
                 "in the select launch)",
                 [&] { return launch_down_mfma(s, a); });
  if (use_multi)
    return timed(s, kTimerDown,
                 "runs-multi-down: down_runs_multi_kernel (each expert's down rows for all its "
                 "tokens on f16 MFMA) + combine_kernel (residual + ranks in order)",
                 [&] {
                   if (int st2 = launch_down_runs_multi(s, a, quant)) return st2;
                   return launch_topk_combine(s, nullptr, a.residual, a.y, nullptr, size_t(a.T),
                                              size_t(a.H), size_t(a.k), a.out);
                 });
  if (use_runs_down)
    return timed(s, kTimerDown,
                 "runs-down: down_runs_kernel (routed down on f16 MFMA + combine; shared down "
                 "in the select launch)",
                 [&] { return launch_down_runs(s, a, quant); });
  return timed(s, kTimerDown, "down8: down8_kernel (routed + Q8_0 shared down + combine)", [&] {
    switch (quant) {
      case INFERNO_Q2_K: launch_down<INFERNO_Q2_K>(s, a); break;
      case INFERNO_Q3_K: launch_down<INFERNO_Q3_K>(s, a); break;
      default: launch_down<INFERNO_Q4_K>(s, a); break;
    }
    INF_LAUNCHED();
    return INFERNO_OK;
  });
}

}  // namespace inferno
