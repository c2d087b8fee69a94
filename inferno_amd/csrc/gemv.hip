// Grouped dequant-GEMV for decode-sized expert groups.
//
// Work item = (active expert slot, 32 output rows). A 256-thread workgroup is
// four wavefronts; each wavefront owns 8 rows and gives every row 8 lanes.
// The wavefront sweeps the rows' super-blocks in order, so at each step the
// 8 rows share one block column and the lanes of a row split its 256 values
// into four runs of 8. The activations of up to NT tokens of the expert's
// group sit in LDS as fp32; quantised bytes are read straight from HBM once
// per workgroup and decoded in registers.
//
// Epilogues: gate/up -> silu(g)*u*w_route (crates/backend/src/metal/kernels/
// gguf_moe_kernels.metal:340-400, Laguna folding of the routing weight);
// down -> per-assignment rows; dense down -> residual_a + residual_b + value
// (q2_kernels.metal:2066-2131), where residual_a may be the rank-order sum of
// the per-assignment routed rows (moe_kernels.metal:210-238).
#include "gemv_common.hpp"

namespace inferno {
namespace {

constexpr int kRowsPerWave = 8;
constexpr int kRowsPerBlock = 4 * kRowsPerWave;

__device__ __forceinline__ uint32_t ld32(const uint8_t* p) { return ld_u1(p); }
__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xffu; }

// Value offsets (within the 256-value super-block) of the lane's four runs
// of eight values, for lane-in-row `sub` (0..7).
template <int Q>
__device__ __forceinline__ void run_offsets(int sub, int off[4]) {
  if constexpr (Q == INFERNO_Q2_K) {
    int h = sub >> 2, s = (sub >> 1) & 1, c = sub & 1;
#pragma unroll
    for (int p = 0; p < 4; ++p) off[p] = 128 * h + 32 * p + 16 * s + 8 * c;
  } else if constexpr (Q == INFERNO_Q3_K) {
    int n = sub >> 2, half = (sub >> 1) & 1, c = sub & 1;
#pragma unroll
    for (int j = 0; j < 4; ++j) off[j] = 16 * (8 * n + 2 * j + half) + 8 * c;
  } else if constexpr (Q == INFERNO_Q4_K) {
    int chunk = sub >> 1, u = sub & 1;
    off[0] = 64 * chunk + 16 * u;
    off[1] = off[0] + 8;
    off[2] = 64 * chunk + 32 + 16 * u;
    off[3] = off[2] + 8;
  } else if constexpr (Q == INFERNO_Q6_K) {
    int half = sub >> 2, i0 = 8 * (sub & 3);
#pragma unroll
    for (int q = 0; q < 4; ++q) off[q] = 128 * half + 32 * q + i0;
  } else {  // Q8_0: lane = one 32-value block
#pragma unroll
    for (int j = 0; j < 4; ++j) off[j] = 32 * sub + 8 * j;
  }
}

// Decodes the lane's 32 weights of super-block `sb` into w[run][i].
template <int Q>
__device__ __forceinline__ void decode_lane(const uint8_t* __restrict__ sb, int sub,
                                            float w[4][8]) {
  if constexpr (Q == INFERNO_Q2_K) {
    int h = sub >> 2, s = (sub >> 1) & 1, c = sub & 1;
    const uint8_t* q = sb + 16 + 32 * h + 16 * s + 8 * c;
    uint32_t q0 = ld32(q), q1 = ld32(q + 4);
    uint32_t s0 = ld32(sb + 8 * h), s1 = ld32(sb + 8 * h + 4);
    uint32_t dd = ld32(sb + 80);
    float d = f16_bits_to_f32(uint16_t(dd)), dmin = f16_bits_to_f32(uint16_t(dd >> 16));
    uint32_t scb[4] = {byte_of(s0, s), byte_of(s0, 2 + s), byte_of(s1, s), byte_of(s1, 2 + s)};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      float sc = d * float(scb[p] & 15u), mn = dmin * float(scb[p] >> 4);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t byte = byte_of(i < 4 ? q0 : q1, i & 3);
        w[p][i] = sc * float((byte >> (2 * p)) & 3u) - mn;
      }
    }
  } else if constexpr (Q == INFERNO_Q3_K) {
    int n = sub >> 2, half = (sub >> 1) & 1, c = sub & 1;
    const uint8_t* q = sb + 32 + 32 * n + 16 * half + 8 * c;
    const uint8_t* hm = sb + 16 * half + 8 * c;
    uint32_t q0 = ld32(q), q1 = ld32(q + 4), h0 = ld32(hm), h1 = ld32(hm + 4);
    const uint8_t* sc = sb + 96;
    float d = f16_bits_to_f32(load_le16(sb + 108));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int g = 8 * n + 2 * j + half;
      uint32_t lo = (g < 8) ? (sc[g % 8] & 15u) : (sc[g % 8] >> 4);
      uint32_t hi = (sc[8 + g % 4] >> (2 * (g / 4))) & 3u;
      float gs = d * (float(int(lo | (hi << 4))) - 32.0f);
      int hb = 4 * n + j;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t qb = byte_of(i < 4 ? q0 : q1, i & 3);
        uint32_t hbyte = byte_of(i < 4 ? h0 : h1, i & 3);
        int v = int((qb >> (2 * j)) & 3u) - (((hbyte >> hb) & 1u) ? 0 : 4);
        w[j][i] = gs * float(v);
      }
    }
  } else if constexpr (Q == INFERNO_Q4_K) {
    int chunk = sub >> 1, u = sub & 1;
    const uint8_t* q = sb + 16 + 32 * chunk + 16 * u;
    uint32_t qw[4] = {ld32(q), ld32(q + 4), ld32(q + 8), ld32(q + 12)};
    uint32_t dd = ld32(sb);
    float d = f16_bits_to_f32(uint16_t(dd)), dmin = f16_bits_to_f32(uint16_t(dd >> 16));
    const uint8_t* s = sb + 4;
    float scf[2], mnf[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      int g = 2 * chunk + k;
      uint32_t sc, m;
      if (g < 4) {
        sc = s[g] & 63u;
        m = s[g + 4] & 63u;
      } else {
        sc = (s[g + 4] & 15u) | ((s[g - 4] >> 6) << 4);
        m = (s[g + 4] >> 4) | ((s[g] >> 6) << 4);
      }
      scf[k] = d * float(sc);
      mnf[k] = dmin * float(m);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int k = j >> 1, base = (j & 1) * 8;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t byte = byte_of(qw[(base + i) >> 2], (base + i) & 3);
        w[j][i] = scf[k] * float((byte >> (4 * k)) & 15u) - mnf[k];
      }
    }
  } else if constexpr (Q == INFERNO_Q6_K) {
    int half = sub >> 2, i0 = 8 * (sub & 3);
    const uint8_t* qa = sb + 64 * half + i0;
    const uint8_t* qb = qa + 32;
    const uint8_t* qh = sb + 128 + 32 * half + i0;
    uint32_t a0 = ld32(qa), a1 = ld32(qa + 4), b0 = ld32(qb), b1 = ld32(qb + 4);
    uint32_t h0 = ld32(qh), h1 = ld32(qh + 4);
    float d = f16_bits_to_f32(load_le16(sb + 208));
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      float sc = d * float(int8_t(sb[192 + 8 * half + (i0 >> 4) + 2 * qq]));
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t lowb = (qq & 1) ? byte_of(i < 4 ? b0 : b1, i & 3) : byte_of(i < 4 ? a0 : a1, i & 3);
        uint32_t l = (qq >= 2) ? (lowb >> 4) : (lowb & 15u);
        uint32_t hh = (byte_of(i < 4 ? h0 : h1, i & 3) >> (2 * qq)) & 3u;
        w[qq][i] = sc * (float(int(l | (hh << 4))) - 32.0f);
      }
    }
  } else {  // Q8_0
    const uint8_t* b = sb + 34 * sub;
    float d = f16_bits_to_f32(load_le16(b));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t v0 = ld32(b + 2 + 8 * j), v1 = ld32(b + 6 + 8 * j);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint32_t byte = byte_of(i < 4 ? v0 : v1, i & 3);
        w[j][i] = d * float(int8_t(byte));
      }
    }
  }
}

template <int Q, int MODE, typename XT, int NT>
__global__ void __launch_bounds__(256) gemv_kernel(GemvArgs p) {
  extern __shared__ float xs[];  // [NT][K]
  constexpr bool kGateUp = MODE == kGateUpRouted || MODE == kGateUpDense;
  constexpr bool kRouted = MODE == kGateUpRouted || MODE == kDownRouted;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane & 7;
  const int row = blockIdx.x * kRowsPerBlock + wave * kRowsPerWave + (lane >> 3);
  const bool row_ok = row < p.rows;
  const int rowc = row_ok ? row : p.rows - 1;

  uint32_t e = 0, lo = 0, hi = uint32_t(p.n_tokens);
  if constexpr (kRouted) {
    if (blockIdx.y >= p.active[0]) return;
    e = p.active[1 + blockIdx.y];
    lo = p.offsets[e];
    hi = p.offsets[e + 1];
  }
  const int SB = Q == INFERNO_Q8_0 ? 272 : (Q == INFERNO_Q2_K ? 84 : Q == INFERNO_Q3_K ? 110 : Q == INFERNO_Q4_K ? 144 : 210);
  const int bpr = p.K / kKBlock;
  const size_t row_bytes = size_t(bpr) * SB;
  const uint8_t* r0 = p.w0 + size_t(e) * p.expert_stride + size_t(rowc) * row_bytes;
  const uint8_t* r1 = kGateUp ? p.w1 + size_t(e) * p.expert_stride + size_t(rowc) * row_bytes : nullptr;
  int off[4];
  run_offsets<Q>(sub, off);

  for (uint32_t c0 = lo; c0 < hi; c0 += NT) {
    const int nt = int(min(uint32_t(NT), hi - c0));
    // stage activations of this chunk
    for (int t = 0; t < nt; ++t) {
      uint32_t src;
      if constexpr (MODE == kGateUpRouted) src = p.sorted[c0 + t] / uint32_t(p.k);  // token
      else if constexpr (MODE == kDownRouted) src = p.sorted[c0 + t];               // assignment
      else src = c0 + t;
      const XT* xrow = static_cast<const XT*>(p.x) + size_t(src) * p.K;
      for (int i = tid; i < p.K; i += 256) xs[t * p.K + i] = to_f32<XT>(xrow[i]);
    }
    __syncthreads();
    float acc0[NT], acc1[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc0[t] = acc1[t] = 0.f;
    for (int b = 0; b < bpr; ++b) {
      float w[4][8], u[4][8];
      decode_lane<Q>(r0 + size_t(b) * SB, sub, w);
      if constexpr (kGateUp) decode_lane<Q>(r1 + size_t(b) * SB, sub, u);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if (t < nt) {
          const float* xb = xs + t * p.K + b * kKBlock;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float4 xa = *reinterpret_cast<const float4*>(xb + off[j]);
            float4 xc = *reinterpret_cast<const float4*>(xb + off[j] + 4);
            float xv[8] = {xa.x, xa.y, xa.z, xa.w, xc.x, xc.y, xc.z, xc.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              acc0[t] += w[j][i] * xv[i];
              if constexpr (kGateUp) acc1[t] += u[j][i] * xv[i];
            }
          }
        }
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t < nt) {
        float g = acc0[t], v = acc1[t];
#pragma unroll
        for (int m = 1; m < 8; m <<= 1) {
          g += __shfl_xor(g, m, kWave);
          if constexpr (kGateUp) v += __shfl_xor(v, m, kWave);
        }
        if (sub == 0 && row_ok) {
          if constexpr (MODE == kGateUpRouted) {
            uint32_t a = p.sorted[c0 + t];
            p.out[size_t(a) * p.rows + row] = silu(g) * v * p.route_w[a];
          } else if constexpr (MODE == kGateUpDense) {
            p.out[size_t(c0 + t) * p.rows + row] = silu(g) * v;
          } else if constexpr (MODE == kDownRouted) {
            uint32_t a = p.sorted[c0 + t];
            p.out[size_t(a) * p.rows + row] = g;
          } else {
            size_t o = size_t(c0 + t) * p.rows + row;
            float ra = 0.f;
            if (p.yk) {
              for (int r = 0; r < p.k; ++r) ra += p.yk[(size_t(c0 + t) * p.k + r) * p.rows + row];
            } else if (p.res_a) {
              ra = p.res_a[o];
            }
            float rb = p.res_b ? p.res_b[o] : 0.f;
            p.out[o] = ra + rb + g;
          }
        }
      }
    }
    __syncthreads();
  }
}

template <int Q, int MODE, typename XT>
int launch_q(hipStream_t s, const GemvArgs& a, int n_slots, int nt) {
  dim3 grid(unsigned((a.rows + kRowsPerBlock - 1) / kRowsPerBlock), unsigned(n_slots));
  if (nt <= 1) {
    size_t lds = size_t(a.K) * sizeof(float);
    gemv_kernel<Q, MODE, XT, 1><<<grid, 256, lds, s>>>(a);
  } else if (nt == 2) {
    size_t lds = 2 * size_t(a.K) * sizeof(float);
    gemv_kernel<Q, MODE, XT, 2><<<grid, 256, lds, s>>>(a);
  } else {
    size_t lds = 4 * size_t(a.K) * sizeof(float);
    gemv_kernel<Q, MODE, XT, 4><<<grid, 256, lds, s>>>(a);
  }
  INF_LAUNCHED();
  return INFERNO_OK;
}

template <int MODE, typename XT>
int launch_mode(hipStream_t s, int quant, const GemvArgs& a, int n_slots, int nt) {
  switch (quant) {
    case INFERNO_Q2_K: return launch_q<INFERNO_Q2_K, MODE, XT>(s, a, n_slots, nt);
    case INFERNO_Q3_K: return launch_q<INFERNO_Q3_K, MODE, XT>(s, a, n_slots, nt);
    case INFERNO_Q4_K: return launch_q<INFERNO_Q4_K, MODE, XT>(s, a, n_slots, nt);
    case INFERNO_Q6_K: return launch_q<INFERNO_Q6_K, MODE, XT>(s, a, n_slots, nt);
    case INFERNO_Q8_0: return launch_q<INFERNO_Q8_0, MODE, XT>(s, a, n_slots, nt);
  }
  set_error("unsupported quant kind for GEMV");
  return INFERNO_ERR_INVALID;
}

// Tokens per LDS chunk: every group of a T=1 step has one member; otherwise
// as many as fit in 32 KiB of staged activations (at most 4).
int pick_nt(size_t T, size_t bytes_per_row) {
  if (T <= 1) return 1;
  size_t fit = (32 * 1024) / bytes_per_row;
  if (fit >= 4) return 4;
  if (fit >= 2) return 2;
  return 1;
}

// Runs MODE through the packed-f16 kernel when the format has one (staging
// the activation rows first unless `staged_ready`), else through the fp32
// reference-layout kernel.
template <int MODE>
int run(hipStream_t s, int quant, GemvArgs& a, const void* x, int x_dtype, size_t stage_rows,
        uint32_t* stage, bool staged_ready, size_t T, int n_slots) {
  if (dot2_supported(quant)) {
    if (!staged_ready) {
      int st = launch_stage(s, x, x_dtype, stage_rows, size_t(a.K), stage);
      if (st) return st;
    }
    const size_t row_bytes = staged_bytes(1, size_t(a.K), x_dtype);
    return launch_dot2<MODE>(s, quant, a, stage, x_dtype, n_slots, pick_nt(T, row_bytes));
  }
  const int nt = pick_nt(T, size_t(a.K) * sizeof(float));
  if (x_dtype == INFERNO_BF16) return launch_mode<MODE, uint16_t>(s, quant, a, n_slots, nt);
  return launch_mode<MODE, float>(s, quant, a, n_slots, nt);
}

}  // namespace

size_t gemv_stage_bytes(int quant, size_t rows, size_t K, int x_dtype) {
  return dot2_supported(quant) ? staged_bytes(rows, K, x_dtype) : 0;
}

int launch_gemv_gate_up_routed(hipStream_t s, int quant, const void* gate, const void* up,
                               const void* x, int x_dtype, uint32_t* stage, bool staged_ready,
                               const uint32_t* offsets, const uint32_t* sorted,
                               const uint32_t* active, const float* route_w, size_t T, size_t k,
                               size_t E, size_t H, size_t I, float* h_out,
                               uint32_t* h_staged_out) {
  GemvArgs a{};
  a.out_staged = h_staged_out;
  a.w0 = static_cast<const uint8_t*>(gate);
  a.w1 = static_cast<const uint8_t*>(up);
  a.x = x;
  a.offsets = offsets;
  a.sorted = sorted;
  a.active = active;
  a.route_w = route_w;
  a.out = h_out;
  a.rows = int(I);
  a.K = int(H);
  a.k = int(k);
  a.expert_stride = I * (H / kKBlock) * size_t(super_bytes(quant));
  return run<kGateUpRouted>(s, quant, a, x, x_dtype, T, stage, staged_ready, T,
                            int(std::min(E, T * k)));
}

int launch_gemv_down_routed(hipStream_t s, int quant, const void* down, const float* h,
                            uint32_t* stage, bool staged_ready, const uint32_t* offsets,
                            const uint32_t* sorted, const uint32_t* active, size_t T, size_t k,
                            size_t E, size_t H, size_t I, float* y_out) {
  GemvArgs a{};
  a.w0 = static_cast<const uint8_t*>(down);
  a.x = h;
  a.offsets = offsets;
  a.sorted = sorted;
  a.active = active;
  a.out = y_out;
  a.rows = int(H);
  a.K = int(I);
  a.k = int(k);
  a.expert_stride = H * (I / kKBlock) * size_t(super_bytes(quant));
  return run<kDownRouted>(s, quant, a, h, INFERNO_F32, T * k, stage, staged_ready, T,
                          int(std::min(E, T * k)));
}

int launch_gemv_gate_up_dense(hipStream_t s, int quant, const void* gate, const void* up,
                              const void* x, int x_dtype, uint32_t* stage, bool staged_ready,
                              size_t T, size_t H, size_t I, float* out, uint32_t* out_staged) {
  GemvArgs a{};
  a.out_staged = out_staged;
  a.w0 = static_cast<const uint8_t*>(gate);
  a.w1 = static_cast<const uint8_t*>(up);
  a.x = x;
  a.out = out;
  a.rows = int(I);
  a.K = int(H);
  a.n_tokens = int(T);
  return run<kGateUpDense>(s, quant, a, x, x_dtype, T, stage, staged_ready, T, 1);
}

int launch_gemv_down_dense(hipStream_t s, int quant, const void* w, const float* input,
                           uint32_t* stage, bool staged_ready, const float* yk, size_t k,
                           const float* res_a, const float* res_b, size_t T, size_t In, size_t O,
                           float* out) {
  GemvArgs a{};
  a.w0 = static_cast<const uint8_t*>(w);
  a.x = input;
  a.yk = yk;
  a.k = int(k);
  a.res_a = res_a;
  a.res_b = res_b;
  a.out = out;
  a.rows = int(O);
  a.K = int(In);
  a.n_tokens = int(T);
  return run<kDownDense>(s, quant, a, input, INFERNO_F32, T, stage, staged_ready, T, 1);
}

}  // namespace inferno
