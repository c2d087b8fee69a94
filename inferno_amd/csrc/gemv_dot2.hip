// Separate-kernel packed-f16 GEMV path (Q2_K, Q3_K, Q4_K, Q8_0): one launch
// per stage. Used by the stage-level entry points, inferno_gguf_moe and the
// Q8_0 shared-expert entry points; the decode layer uses the fused path in
// decode.hip built from the same tile functions (dot2_formats.hpp).
//
// Work item: 16 rows of one expert (gate and up together for the SwiGLU
// stage) for up to NT activation rows of that expert's group. Semantics
// follow crates/backend/src/metal/kernels/gguf_moe_kernels.metal:340-565
// (gate/up SwiGLU with the routing weight folded, down per assignment),
// laguna_xs_kernels.metal:1578-1642 (Q4_K) and q2_kernels.metal:2066-2235
// (Q8_0 shared expert, residual_a + residual_b + value).
#include "dot2_formats.hpp"

namespace inferno {
namespace {

// One thread per 16-value run: stages rows of x into the packed layout.
template <typename XT, bool SPLIT>
__global__ void __launch_bounds__(256)
    stage_runs_kernel(const XT* __restrict__ x, int rows, int K, uint32_t* __restrict__ staged) {
  const int runs = K / 16;
  const size_t id = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (id >= size_t(rows) * runs) return;
  const int r = int(id / runs), run = int(id % runs);
  const XT* src = x + size_t(r) * K + run * 16;
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = to_f32(src[i]);
  stage_run<SPLIT>(v, staged + size_t(r) * staged_stride(K, SPLIT), K, run);
}

template <int Q, int MODE, int NT, bool SPLIT>
__device__ __forceinline__ void gemv_body(const GemvArgs& p, const uint32_t* __restrict__ staged) {
  constexpr bool kGateUp = MODE == kGateUpRouted || MODE == kGateUpDense;
  constexpr bool kRouted = MODE == kGateUpRouted || MODE == kDownRouted;
  constexpr int kMats = kGateUp ? 2 : 1;
  extern __shared__ uint32_t smem[];
  const int K = p.K;
  const int S = staged_stride(K, SPLIT);
  uint32_t* xs = smem;                                         // NT * S
  float* part = reinterpret_cast<float*>(smem + NT * S);      // tile_part_floats(NT)
  float* res = part + tile_part_floats(NT);                    // 2 * kRows * NT

  const int tid = threadIdx.x, lane = tid & 63;
  const int slot = lane >> 2;
  const int tile = blockIdx.x;
  const int row = tile * kRows + slot;
  const int rowc = row < p.rows ? row : p.rows - 1;

  uint32_t e = 0, lo = 0, hi = uint32_t(p.n_tokens);
  if constexpr (kRouted) {
    if (blockIdx.y >= p.active[0]) return;
    e = p.active[1 + blockIdx.y];
    lo = p.offsets[e];
    hi = p.offsets[e + 1];
  }
  const size_t row_bytes = size_t(K / kKBlock) * Fmt<Q>::kBytes;
  const uint8_t* base0 = p.w0 + size_t(e) * p.expert_stride + size_t(rowc) * row_bytes;
  const uint8_t* base1 =
      kGateUp ? p.w1 + size_t(e) * p.expert_stride + size_t(rowc) * row_bytes : nullptr;

  TileDot<Q, kMats, NT, SPLIT> td(base0, base1, K);
  for (uint32_t c0 = lo; c0 < hi; c0 += NT) {
    const int nt = int(min(uint32_t(NT), hi - c0));
    td.prefetch();
    copy_rows_to_lds(xs, S, nt, [&](int t) {
      uint32_t src = c0 + uint32_t(t);
      if constexpr (MODE == kGateUpRouted) src = p.sorted[src] / uint32_t(p.k);
      else if constexpr (MODE == kDownRouted) src = p.sorted[src];
      return staged + size_t(src) * S;
    });
    __syncthreads();
    td.run(xs, S, nt, part, res);
    if constexpr (kGateUp) {
      // wave t (< nt) writes activation t's 16 outputs and staged run
      const int t = tid >> 6;
      if (t < nt && (tid & 63) < 16) {
        uint32_t a = c0 + uint32_t(t);
        float w = 1.0f;
        if constexpr (MODE == kGateUpRouted) {
          a = p.sorted[a];
          w = p.route_w[a];
        }
        swiglu_tile_out(res, NT, t, w, p.out ? p.out + size_t(a) * p.rows : nullptr,
                        p.out_staged ? p.out_staged + size_t(a) * staged_stride(p.rows, true)
                                     : nullptr,
                        p.rows, tile);
      }
    } else if (tid < kRows * NT) {
      const int s = tid / NT, t = tid % NT;
      const int r = tile * kRows + s;
      if (t < nt && r < p.rows) {
        const float g = res[s * NT + t];
        if constexpr (MODE == kDownRouted) {
          p.out[size_t(p.sorted[c0 + t]) * p.rows + r] = g;
        } else {
          const size_t o = size_t(c0 + t) * p.rows + r;
          float ra = 0.f;
          if (p.yk) {
            for (int rk = 0; rk < p.k; ++rk) ra += p.yk[(size_t(c0 + t) * p.k + rk) * p.rows + r];
          } else if (p.res_a) {
            ra = p.res_a[o];
          }
          p.out[o] = ra + (p.res_b ? p.res_b[o] : 0.f) + g;
        }
      }
    }
    __syncthreads();
  }
}

// Single-activation groups (decode) are held to 128 VGPRs so four
// workgroups fit per CU; multi-activation groups trade occupancy for
// accumulators.
template <int Q, int MODE, bool SPLIT>
__global__ void __launch_bounds__(256)
    __attribute__((amdgpu_waves_per_eu(Occupancy<Q, SPLIT>::value, 8))) gemv1_kernel(GemvArgs p, const uint32_t* __restrict__ staged) {
  gemv_body<Q, MODE, 1, SPLIT>(p, staged);
}

template <int Q, int MODE, int NT, bool SPLIT>
__global__ void __launch_bounds__(256) gemvn_kernel(GemvArgs p,
                                                    const uint32_t* __restrict__ staged) {
  gemv_body<Q, MODE, NT, SPLIT>(p, staged);
}

template <int Q, int MODE, int NT, bool SPLIT>
int launch_nt(hipStream_t s, const GemvArgs& a, const uint32_t* staged, int n_slots) {
  dim3 grid(unsigned((a.rows + kRows - 1) / kRows), unsigned(n_slots));
  const size_t lds = (size_t(NT) * staged_stride(a.K, SPLIT) + tile_part_floats(NT) +
                      2 * kRows * NT) * 4;
  if (lds > 160 * 1024) {
    set_error("activation row too long for the LDS staging buffer");
    return INFERNO_ERR_INVALID;
  }
  if constexpr (NT == 1)
    gemv1_kernel<Q, MODE, SPLIT><<<grid, 256, lds, s>>>(a, staged);
  else
    gemvn_kernel<Q, MODE, NT, SPLIT><<<grid, 256, lds, s>>>(a, staged);
  INF_LAUNCHED();
  return INFERNO_OK;
}

template <int Q, int MODE, bool SPLIT>
int launch_q(hipStream_t s, const GemvArgs& a, const uint32_t* staged, int n_slots, int nt) {
  if (nt <= 1) return launch_nt<Q, MODE, 1, SPLIT>(s, a, staged, n_slots);
  if (nt == 2) return launch_nt<Q, MODE, 2, SPLIT>(s, a, staged, n_slots);
  return launch_nt<Q, MODE, 4, SPLIT>(s, a, staged, n_slots);
}

template <int MODE, bool SPLIT>
int launch_fmt(hipStream_t s, int quant, const GemvArgs& a, const uint32_t* staged, int n_slots,
               int nt) {
  switch (quant) {
    case INFERNO_Q2_K: return launch_q<INFERNO_Q2_K, MODE, SPLIT>(s, a, staged, n_slots, nt);
    case INFERNO_Q3_K: return launch_q<INFERNO_Q3_K, MODE, SPLIT>(s, a, staged, n_slots, nt);
    case INFERNO_Q4_K: return launch_q<INFERNO_Q4_K, MODE, SPLIT>(s, a, staged, n_slots, nt);
    case INFERNO_Q8_0: return launch_q<INFERNO_Q8_0, MODE, SPLIT>(s, a, staged, n_slots, nt);
  }
  set_error("quant kind has no packed-f16 GEMV");
  return INFERNO_ERR_INVALID;
}

}  // namespace

bool dot2_supported(int quant) {
  return quant == INFERNO_Q2_K || quant == INFERNO_Q3_K || quant == INFERNO_Q4_K ||
         quant == INFERNO_Q8_0;
}

size_t staged_bytes(size_t rows, size_t K, int x_dtype) {
  return rows * size_t(staged_stride(int(K), x_dtype == INFERNO_F32)) * 4;
}

int launch_stage(hipStream_t s, const void* x, int x_dtype, size_t rows, size_t K,
                 uint32_t* staged) {
  const size_t n = rows * (K / 16);
  if (n == 0) return INFERNO_OK;
  const unsigned grid = unsigned((n + 255) / 256);
  if (x_dtype == INFERNO_BF16)
    stage_runs_kernel<uint16_t, false><<<grid, 256, 0, s>>>(static_cast<const uint16_t*>(x),
                                                            int(rows), int(K), staged);
  else
    stage_runs_kernel<float, true><<<grid, 256, 0, s>>>(static_cast<const float*>(x), int(rows),
                                                        int(K), staged);
  INF_LAUNCHED();
  return INFERNO_OK;
}

template <int MODE>
int launch_dot2(hipStream_t s, int quant, const GemvArgs& a, const uint32_t* staged, int x_dtype,
                int n_slots, int nt) {
  if (x_dtype == INFERNO_F32) return launch_fmt<MODE, true>(s, quant, a, staged, n_slots, nt);
  return launch_fmt<MODE, false>(s, quant, a, staged, n_slots, nt);
}

template int launch_dot2<kGateUpRouted>(hipStream_t, int, const GemvArgs&, const uint32_t*, int,
                                        int, int);
template int launch_dot2<kGateUpDense>(hipStream_t, int, const GemvArgs&, const uint32_t*, int,
                                       int, int);
template int launch_dot2<kDownRouted>(hipStream_t, int, const GemvArgs&, const uint32_t*, int,
                                      int, int);
template int launch_dot2<kDownDense>(hipStream_t, int, const GemvArgs&, const uint32_t*, int,
                                     int, int);

}  // namespace inferno
