// RMSNorm of one row by one 1024-thread workgroup, in a fixed summation
// order (reference_rms_norm_f32, crates/backend/src/backend.rs:10211-10257:
// x / sqrt(sum x^2 / H + eps) * w). Shared by the RMSNorm launch and the
// fused RMSNorm -> router launch, so both give the same bits for a row.
//
// Rows of a multiple of 4 values up to 32768 are read as float4s all issued
// at once (one memory round trip), the squares summed per thread, per
// wavefront (butterfly) and over the 16 wavefronts in order; other widths
// take a strided scalar loop.
#pragma once
#include "common.hpp"

namespace inferno {

constexpr int kNormThreads = 1024;
constexpr int kNormVec = 8;  // float4s per thread held in registers

// emit(i, v) receives every normalised value v of position i (each once, by
// one thread). `part` is LDS of kNormThreads / 64 + 1 floats. Every thread
// of the workgroup must call it; it contains two barriers.
template <typename Emit>
__device__ __forceinline__ void rms_norm_row(const float* __restrict__ row,
                                             const float* __restrict__ w, size_t H, float eps,
                                             float* part, Emit emit) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool vec = H % 4 == 0 && H <= size_t(4 * kNormThreads * kNormVec);
  float4 v[kNormVec];
  float s = 0.f;
  if (vec) {
    const float4* r4 = reinterpret_cast<const float4*>(row);
#pragma unroll
    for (int j = 0; j < kNormVec; ++j) {
      const size_t i = size_t(j) * kNormThreads + tid;
      v[j] = i < H / 4 ? r4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int j = 0; j < kNormVec; ++j) {
      s += v[j].x * v[j].x;
      s += v[j].y * v[j].y;
      s += v[j].z * v[j].z;
      s += v[j].w * v[j].w;
    }
  } else {
    for (size_t i = tid; i < H; i += kNormThreads) s += row[i] * row[i];
  }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) s += __shfl_xor(s, m, 64);
  if (lane == 0) part[wave] = s;
  __syncthreads();
  if (tid == 0) {
    float t = 0.f;
    for (int i = 0; i < kNormThreads / 64; ++i) t += part[i];
    part[kNormThreads / 64] = sqrtf(t / float(H) + eps);
  }
  __syncthreads();
  const float scale = part[kNormThreads / 64];
  if (vec) {
    const float4* w4 = reinterpret_cast<const float4*>(w);
#pragma unroll
    for (int j = 0; j < kNormVec; ++j) {
      const size_t i = size_t(j) * kNormThreads + tid;
      if (i < H / 4) {
        const float4 g = w4[i];
        emit(4 * i, v[j].x / scale * g.x);
        emit(4 * i + 1, v[j].y / scale * g.y);
        emit(4 * i + 2, v[j].z / scale * g.z);
        emit(4 * i + 3, v[j].w / scale * g.w);
      }
    }
  } else {
    for (size_t i = tid; i < H; i += kNormThreads) emit(i, row[i] / scale * w[i]);
  }
}

}  // namespace inferno
