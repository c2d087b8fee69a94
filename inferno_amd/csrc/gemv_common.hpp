// Shared pieces of the GEMV kernels: argument block, modes, load helpers.
#pragma once
#include "kernels.hpp"

namespace inferno {

enum GemvMode { kGateUpRouted = 0, kGateUpDense = 1, kDownRouted = 2, kDownDense = 3 };

struct GemvArgs {
  const uint8_t* w0;        // gate (gate/up modes) or down
  const uint8_t* w1;        // up (gate/up modes)
  const void* x;            // [tokens or assignments, K]
  const uint32_t* offsets;  // [E+1] (routed)
  const uint32_t* sorted;   // [A]   (routed)
  const uint32_t* active;   // [1+E] (routed)
  const float* route_w;     // [A]   (routed gate/up)
  float* out;
  uint32_t* out_staged;     // gate/up: also write the output rows staged (fp32 layout) or null
  const float* yk;          // dense down: per-assignment routed rows [T*k, rows] or null
  const float* res_a;       // dense down: residual_a or null (ignored when yk set)
  const float* res_b;       // dense down: residual_b or null
  int rows;                 // output rows per expert
  int K;                    // reduction length
  int k;                    // top-k (routed / yk)
  int n_tokens;             // dense: T
  size_t expert_stride;     // bytes per expert matrix
};

// Unaligned vector loads: gfx950 runs with unaligned global access enabled,
// so a 16-byte load only needs the hardware's dword-or-better handling.
typedef uint32_t u32x4_u __attribute__((ext_vector_type(4), aligned(1)));
typedef uint32_t u32x2_u __attribute__((ext_vector_type(2), aligned(1)));
typedef uint32_t u32_u __attribute__((aligned(1)));

__device__ __forceinline__ uint4 ld_u4(const uint8_t* p) {
  u32x4_u v = *reinterpret_cast<const u32x4_u*>(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld_u2(const uint8_t* p) {
  u32x2_u v = *reinterpret_cast<const u32x2_u*>(p);
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ld_u1(const uint8_t* p) {
  return *reinterpret_cast<const u32_u*>(p);
}

__device__ __forceinline__ float f16_bits_to_f32_fast(uint16_t h) {
  return float(__builtin_bit_cast(_Float16, h));
}

template <typename XT>
__device__ __forceinline__ float to_f32(XT v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) {
  return v;
}
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) {
  return bf16_bits_to_f32(v);
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

bool dot2_supported(int quant);
size_t staged_bytes(size_t rows, size_t K, int x_dtype);
int launch_stage(hipStream_t s, const void* x, int x_dtype, size_t rows, size_t K,
                 uint32_t* staged);
template <int MODE>
int launch_dot2(hipStream_t s, int quant, const GemvArgs& a, const uint32_t* staged, int x_dtype,
                int n_slots, int nt);

}  // namespace inferno
