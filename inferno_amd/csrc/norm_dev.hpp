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

// Sum of squares of one float4 added to s, in a fixed order with explicit
// fused multiply-adds (every kernel that forms an RMSNorm scale uses it, so
// they agree bit for bit).
__device__ __forceinline__ float norm_sq4(float s, float4 v) {
  s = fmaf(v.x, v.x, s);
  s = fmaf(v.y, v.y, s);
  s = fmaf(v.z, v.z, s);
  return fmaf(v.w, v.w, s);
}

// One normalised value: x / scale * w (the division rounded first).
__device__ __forceinline__ float norm_apply(float x, float scale, float w) { return x / scale * w; }

// emit(i, v) receives every normalised value v of position i (each once, by
// one thread). `part` is LDS of kNormThreads / 64 + 1 floats. Every thread
// of the workgroup must call it; it contains two barriers.
template <typename Emit>
__device__ __forceinline__ void rms_norm_row(const float* __restrict__ row,
                                             const float* __restrict__ w, size_t H, float eps,
                                             float* part, Emit emit) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool vec = H % 4 == 0 && H <= size_t(4 * kNormThreads * kNormVec);
  float4 v[kNormVec], g[kNormVec];
  float s = 0.f;
  if (vec) {
    // the row and the weights in one round trip (clamped addresses, so the
    // loads are not held behind the bound checks)
    const float4* r4 = reinterpret_cast<const float4*>(row);
    const float4* w4 = reinterpret_cast<const float4*>(w);
    const size_t n4 = H / 4;
#pragma unroll
    for (int j = 0; j < kNormVec; ++j) {
      const size_t i = size_t(j) * kNormThreads + tid;
      const float4 a = r4[i < n4 ? i : n4 - 1], b = w4[i < n4 ? i : n4 - 1];
      v[j] = i < n4 ? a : make_float4(0.f, 0.f, 0.f, 0.f);
      g[j] = b;
    }
#pragma unroll
    for (int j = 0; j < kNormVec; ++j) s = norm_sq4(s, v[j]);
  } else {
    for (size_t i = tid; i < H; i += kNormThreads) s = fmaf(row[i], row[i], s);
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
#pragma unroll
    for (int j = 0; j < kNormVec; ++j) {
      const size_t i = size_t(j) * kNormThreads + tid;
      if (i < H / 4) {
        emit(4 * i, norm_apply(v[j].x, scale, g[j].x));
        emit(4 * i + 1, norm_apply(v[j].y, scale, g[j].y));
        emit(4 * i + 2, norm_apply(v[j].z, scale, g[j].z));
        emit(4 * i + 3, norm_apply(v[j].w, scale, g[j].w));
      }
    }
  } else {
    for (size_t i = tid; i < H; i += kNormThreads) emit(i, norm_apply(row[i], scale, w[i]));
  }
}

}  // namespace inferno
